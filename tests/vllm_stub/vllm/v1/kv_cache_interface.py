from dataclasses import dataclass

import torch


@dataclass
class AttentionSpec:
    block_size: int
    num_kv_heads: int = 1
    head_size: int = 128
    dtype: torch.dtype = torch.float16
