import enum
from dataclasses import dataclass
from typing import Generic, Optional, Protocol, TypeVar

import torch


class AttentionType:
    DECODER = "decoder"
    ENCODER = "encoder"
    ENCODER_ONLY = "encoder_only"
    ENCODER_DECODER = "encoder_decoder"


class AttentionCGSupport(enum.Enum):
    ALWAYS = 3
    UNIFORM_BATCH = 2
    UNIFORM_SINGLE_TOKEN_DECODE = 1
    NEVER = 0


@dataclass(frozen=True)
class MultipleOf:
    base: int


@dataclass
class CommonAttentionMetadata:
    query_start_loc: torch.Tensor
    seq_lens: torch.Tensor
    num_reqs: int
    num_actual_tokens: int
    max_query_len: int
    max_seq_len: int
    block_table_tensor: torch.Tensor
    slot_mapping: torch.Tensor
    query_start_loc_cpu: Optional[torch.Tensor] = None
    seq_lens_cpu: Optional[torch.Tensor] = None


class AttentionLayer(Protocol):
    _k_scale: torch.Tensor
    _v_scale: torch.Tensor


class AttentionBackend:
    accept_output_buffer: bool = False


class AttentionImpl:
    pass


M = TypeVar("M")


class AttentionMetadataBuilder(Generic[M]):
    def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
        self.kv_cache_spec = kv_cache_spec
        self.layer_names = layer_names
        self.vllm_config = vllm_config
        self.device = device
