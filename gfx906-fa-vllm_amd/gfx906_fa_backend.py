# SPDX-License-Identifier: Apache-2.0
"""vLLM v1 attention backend: Q8_0 paged attention on MI355X (gfx950).

Drop-in for ``extension/gfx906_fa_backend.py`` of the reference: same entry
point (``vllm.general_plugins: gfx906_fa = gfx906_fa_backend:register``,
reference ``extension/setup.py:56-60``), same registration as
``AttentionBackendEnum.CUSTOM`` (lines 536-553), same class names and
``forward`` / ``do_kv_cache_update`` signatures (lines 405-461).

What differs, by design:
  * K **and** V are stored as Q8_0 (the reference keeps V in fp16 and K in a
    side buffer that can go stale, lines 277-314 and 428-434).  The Q8 planes
    live inside vLLM's own per-layer KV tensor, so every write goes through
    ``do_kv_cache_update`` and there is no second copy to fall out of sync.
  * ``forward`` makes one varlen HIP call for decode / prefill / mixed /
    speculative-verify batches and writes ``output`` in place in the model
    dtype (the reference upcasts Q to fp32, pads, and copies back, lines
    478-528).
  * fp16 and bf16 models; head size 128 (the only size the reference's
    launchers accept, ``extension/gfx906_fa_launcher.cu:76-79``); any block
    size that is a multiple of 16.
"""
from __future__ import annotations

import os
from dataclasses import dataclass
from typing import ClassVar

import torch

from vllm.config import VllmConfig
from vllm.config.cache import CacheDType
from vllm.logger import init_logger
from vllm.platforms.interface import DeviceCapability
from vllm.v1.attention.backend import (
    AttentionBackend,
    AttentionCGSupport,
    AttentionImpl,
    AttentionLayer,
    AttentionMetadataBuilder,
    AttentionType,
    CommonAttentionMetadata,
    MultipleOf,
)
from vllm.v1.kv_cache_interface import AttentionSpec

import gfx906_fa
from gfx906_fa_paged import forward_paged, q8_planes

logger = init_logger(__name__)

# kv_cache_dtype of the cache whose pages hold exactly the Q8_0 planes
Q8_CACHE_DTYPE = "q8_0"
_KV_CACHE_DTYPES = ("auto", "float16", "half", "bfloat16", Q8_CACHE_DTYPE)


# -----------------------------------------------------------------------------
# Metadata (reference lines 59-109)
# -----------------------------------------------------------------------------
@dataclass
class Gfx906FAMetadata:
    num_actual_tokens: int
    max_query_len: int
    max_seq_len: int
    query_start_loc: torch.Tensor      # [B+1] int32
    seq_lens: torch.Tensor             # [B]   int32
    block_table: torch.Tensor          # [B, max_num_blocks] int32
    slot_mapping: torch.Tensor         # [num_tokens] int64
    use_cascade: bool = False
    common_prefix_len: int = 0


def workspace_upper_bound(max_num_seqs: int, max_num_tokens: int, heads, max_seq_len: int = -1,
                          image_room: int | None = None) -> int:
    """Attention workspace that covers every batch of up to max_num_seqs
    sequences and max_num_tokens query tokens - any query lengths, any mix of
    decode, speculative-verify and prefill sequences, any context - for each
    layer shape (num_heads, num_kv_heads) in ``heads``: the regions every
    such call needs plus the prefill tile-image room for contexts up to
    max_seq_len (-1: any), capped at ``image_room`` bytes when given (the
    room is optional: prefill workgroups dequantize their own tiles where
    images do not fit)."""
    best = 0
    for hq, hkv in heads:
        i = gfx906_fa.workspace_bound_info(max_num_seqs, max_num_tokens, hq, hkv, max_seq_len)
        img = i["img_bytes"] if image_room is None else min(i["img_bytes"], max(int(image_room), 0))
        best = max(best, i["regions"] + img)
    return best


def image_room_bytes() -> int:
    """The tile-image room the backend reserves at most: GFX906_FA_IMAGE_ROOM_MB
    (default 256 MiB, enough for the images of a 57K-token prompt at 8
    kv-heads; 0 turns prefill tile images off)."""
    try:
        mb = int(os.environ.get("GFX906_FA_IMAGE_ROOM_MB", "256"))
    except ValueError:
        mb = 256
    return max(mb, 0) << 20


def _scheduler_limits(vllm_config) -> tuple[int, int, int] | None:
    """(max_num_seqs, max_num_batched_tokens, max_model_len or -1) of a vLLM
    config, or None where the scheduler limits are not set."""
    sched = getattr(vllm_config, "scheduler_config", None)
    max_seqs = getattr(sched, "max_num_seqs", None)
    max_tokens = getattr(sched, "max_num_batched_tokens", None)
    if not (isinstance(max_seqs, int) and max_seqs > 0 and isinstance(max_tokens, int) and max_tokens > 0):
        return None
    mml = getattr(getattr(vllm_config, "model_config", None), "max_model_len", None)
    return max_seqs, max_tokens, mml if isinstance(mml, int) and mml > 0 else -1


class Gfx906FAMetadataBuilder(AttentionMetadataBuilder[Gfx906FAMetadata]):
    # Graph-capturable for batches of one query length (decode, speculative
    # verify): the kernels read every per-step value from device memory, size
    # their grids from fixed shapes only, allocate nothing and record no
    # memset (the reference is NEVER, extension/gfx906_fa_backend.py:75).
    _cudagraph_support: ClassVar[AttentionCGSupport] = AttentionCGSupport.UNIFORM_BATCH

    def __init__(self, kv_cache_spec: AttentionSpec, layer_names: list[str],
                 vllm_config: VllmConfig, device: torch.device):
        super().__init__(kv_cache_spec, layer_names, vllm_config, device)
        self.block_size = kv_cache_spec.block_size
        # Reserve the shared workspace before any capture, so forward() never
        # allocates inside a graph: the bound over the scheduler's batch
        # limits for every layer shape seen (the Impls are built with the
        # model, before the builders).  The profiling forward has normally
        # reserved it already (so vLLM's memory profile counts it); this
        # covers layer shapes seen only now.
        limits = _scheduler_limits(vllm_config)
        if limits is not None:
            Gfx906FAImpl._limits = limits
        heads = set(Gfx906FAImpl._layer_heads)
        hkv = getattr(kv_cache_spec, "num_kv_heads", None)
        model_config = getattr(vllm_config, "model_config", None)
        if model_config is not None and isinstance(hkv, int) and hkv > 0:
            try:
                heads.add((int(model_config.get_num_attention_heads(vllm_config.parallel_config)), hkv))
            except (AttributeError, TypeError, ValueError):
                pass
        if limits is not None and heads and torch.device(device).type == "cuda":
            Gfx906FAImpl.reserve_workspace(Gfx906FAImpl.bound_bytes(heads, limits), torch.device(device))

    def build_for_cudagraph_capture(self, common_attn_metadata: CommonAttentionMetadata
                                    ) -> Gfx906FAMetadata:
        # a graph captured from here keeps the workspace's raw address: from
        # now on a replaced workspace must stay allocated
        Gfx906FAImpl._captured = True
        return self.build(0, common_attn_metadata)

    def build(self, common_prefix_len: int, common_attn_metadata: CommonAttentionMetadata,
              fast_build: bool = False) -> Gfx906FAMetadata:
        return Gfx906FAMetadata(
            num_actual_tokens=common_attn_metadata.num_actual_tokens,
            max_query_len=common_attn_metadata.max_query_len,
            max_seq_len=common_attn_metadata.max_seq_len,
            query_start_loc=common_attn_metadata.query_start_loc,
            seq_lens=common_attn_metadata.seq_lens,
            block_table=common_attn_metadata.block_table_tensor,
            slot_mapping=common_attn_metadata.slot_mapping,
            use_cascade=(common_prefix_len > 0),
            common_prefix_len=common_prefix_len,
        )


# -----------------------------------------------------------------------------
# Backend (reference lines 115-209)
# -----------------------------------------------------------------------------
class Gfx906FABackend(AttentionBackend):
    accept_output_buffer: bool = True

    supported_dtypes: ClassVar[list[torch.dtype]] = [torch.float16, torch.bfloat16]
    # "auto" / "float16" / "half" / "bfloat16": vLLM allocates the pages in the
    # model dtype and the Q8_0 planes are stored inside them (the first 272 of
    # every 512 bytes per token and kv-head are used).  "q8_0": pages of
    # exactly the Q8_0 planes, 272 bytes per token and kv-head (1.88x the
    # tokens per GiB); needs vLLM to size the page with q8_page_size_bytes().
    supported_kv_cache_dtypes: ClassVar[list[CacheDType]] = ["auto", "float16", "half", "bfloat16",
                                                             Q8_CACHE_DTYPE]

    forward_includes_kv_cache_update: bool = False

    @staticmethod
    def get_supported_kernel_block_sizes() -> list[int | MultipleOf]:
        return [MultipleOf(16)]

    @classmethod
    def supports_block_size(cls, block_size: int | None) -> bool:
        if block_size is None:
            return True
        return block_size % 16 == 0

    @staticmethod
    def get_name() -> str:
        return "CUSTOM"

    @staticmethod
    def get_impl_cls() -> type["Gfx906FAImpl"]:
        return Gfx906FAImpl

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int,
                           cache_dtype_str: str = "auto") -> tuple[int, ...]:
        if block_size % 16 != 0:
            raise ValueError("Block size must be a multiple of 16.")
        if cache_dtype_str == Q8_CACHE_DTYPE:
            # uint8 page = [K plane | V plane], each [Hkv][block_size/16
            # sub-pages][2176 B]; five dims so vLLM's identity stride order
            # applies unchanged
            if head_size != 128:
                raise ValueError("the Q8_0 page layout needs head_size 128")
            return (num_blocks, 2, num_kv_heads, block_size // 16, gfx906_fa.SUBPAGE_BYTES)
        # Same as TritonAttentionBackend, so the allocator is unchanged.
        return (num_blocks, 2, block_size, num_kv_heads, head_size)

    @staticmethod
    def q8_page_size_bytes(block_size: int, num_kv_heads: int, head_size: int = 128) -> int:
        """Bytes of one page of the "q8_0" cache: K and V Q8_0 rows of
        block_size tokens x num_kv_heads, (head_size/32)*34 bytes each
        (extension/gfx906_fa_quant.cu:142-145 sizes the reference's K rows
        the same way).  vLLM's page for this cache dtype must be exactly this
        (a uint8 FullAttentionSpec padded to it)."""
        if block_size % 16 != 0 or head_size != 128:
            raise ValueError("the Q8_0 page layout needs block_size % 16 == 0 and head_size 128")
        return 2 * num_kv_heads * (block_size // 16) * gfx906_fa.SUBPAGE_BYTES

    @staticmethod
    def get_kv_cache_page_size_bytes(block_size: int, num_kv_heads: int, head_size: int,
                                     cache_dtype_str: str, model_dtype: torch.dtype) -> int:
        """Page bytes for either cache layout (what vLLM's KV-cache spec has
        to allocate per block)."""
        if cache_dtype_str == Q8_CACHE_DTYPE:
            return Gfx906FABackend.q8_page_size_bytes(block_size, num_kv_heads, head_size)
        itemsize = torch.empty((), dtype=model_dtype).element_size()
        return 2 * block_size * num_kv_heads * head_size * itemsize

    @staticmethod
    def get_kv_cache_stride_order(include_num_layers_dimension: bool = False) -> tuple[int, ...]:
        if include_num_layers_dimension:
            return (1, 0, 2, 3, 4, 5)
        return (0, 1, 2, 3, 4)

    @staticmethod
    def use_cascade_attention(*args, **kwargs) -> bool:
        return False

    @staticmethod
    def get_builder_cls() -> type["Gfx906FAMetadataBuilder"]:
        return Gfx906FAMetadataBuilder

    @classmethod
    def supports_head_size(cls, head_size: int) -> bool:
        return head_size == 128

    @classmethod
    def supports_mm_prefix(cls) -> bool:
        return False

    @classmethod
    def supports_sink(cls) -> bool:
        return False

    @classmethod
    def supports_attn_type(cls, attn_type: str) -> bool:
        return attn_type == AttentionType.DECODER

    @classmethod
    def supports_alibi_sqrt(cls) -> bool:
        return False

    @classmethod
    def supports_compute_capability(cls, capability: DeviceCapability) -> bool:
        return True


# -----------------------------------------------------------------------------
# Impl (reference lines 215-530)
# -----------------------------------------------------------------------------
class Gfx906FAImpl(AttentionImpl):
    # One attention workspace per worker, shared by all layers (the reference
    # shares its gather buffers the same way, lines 229-230).  Layers run in
    # order on one stream, so reuse is safe.
    _workspace: ClassVar[torch.Tensor | None] = None
    # Workspaces replaced by a larger one after a graph capture.  A captured
    # graph holds the raw address of the workspace it was captured with (the
    # kernels receive pointers, so the graph keeps no reference to the
    # tensor): such a workspace stays allocated for the life of the process,
    # since later replays still write into it.  Before any capture a replaced
    # workspace is simply freed.
    _retired: ClassVar[list[torch.Tensor]] = []
    _captured: ClassVar[bool] = False
    # (num_heads, num_kv_heads) of every layer built, for the workspace bound
    _layer_heads: ClassVar[set[tuple[int, int]]] = set()
    # (max_num_seqs, max_num_batched_tokens, max_model_len) of the scheduler
    _limits: ClassVar[tuple[int, int, int] | None] = None

    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: int,
                 alibi_slopes: list[float] | None, sliding_window: int | None,
                 kv_cache_dtype: str, logits_soft_cap: float | None = None,
                 attn_type: AttentionType = AttentionType.DECODER,
                 kv_sharing_target_layer_name: int | None = None,
                 sinks: torch.Tensor | None = None, use_alibi_sqrt: bool = False) -> None:
        if alibi_slopes is not None:
            raise NotImplementedError("GFX906_FA: alibi_slopes is not supported")
        if sliding_window is not None:
            raise NotImplementedError("GFX906_FA: sliding_window is not supported")
        if logits_soft_cap not in (None, 0, 0.0):
            raise NotImplementedError("GFX906_FA: logits_soft_cap is not supported")
        if sinks is not None:
            raise NotImplementedError("GFX906_FA: sinks are not supported")
        if attn_type != AttentionType.DECODER:
            raise NotImplementedError(f"GFX906_FA: attn_type={attn_type} is not supported")
        if head_size != 128:
            raise NotImplementedError(f"GFX906_FA: head_size={head_size} is not supported (128 only)")
        if num_heads % num_kv_heads != 0:
            raise ValueError("num_heads must be a multiple of num_kv_heads")
        if kv_cache_dtype not in _KV_CACHE_DTYPES:
            raise NotImplementedError(f"GFX906_FA: kv_cache_dtype={kv_cache_dtype} is not supported")
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.num_kv_heads = num_kv_heads
        self.kv_cache_dtype = kv_cache_dtype
        self.attn_type = attn_type
        self.kv_sharing_target_layer_name = kv_sharing_target_layer_name
        self.num_queries_per_kv = num_heads // num_kv_heads
        Gfx906FAImpl._layer_heads.add((num_heads, num_kv_heads))
        if Gfx906FAImpl._limits is None:
            # the scheduler limits of the model being built (set by vLLM
            # around model construction), for the profiling forward
            try:
                from vllm.config import get_current_vllm_config
                Gfx906FAImpl._limits = _scheduler_limits(get_current_vllm_config())
            except (ImportError, AttributeError, TypeError):
                pass

    def fused_output_quant_supported(self, quant_key):
        return False

    def fused_rope_kvcache_supported(self):
        # do_rope_and_kv_cache_update rotates query/key and writes the Q8_0
        # cache in one launch (the reference returns False,
        # extension/gfx906_fa_backend.py:444-445)
        return True

    def do_rope_and_kv_cache_update(self, layer: AttentionLayer, query: torch.Tensor,
                                    key: torch.Tensor, value: torch.Tensor, positions: torch.Tensor,
                                    cos_sin_cache: torch.Tensor, is_neox: bool, kv_cache: torch.Tensor,
                                    layer_slot_mapping: torch.Tensor):
        """vLLM's fused rope + KV-cache update: query [T, Hq*D] / [T, Hq, D]
        and key are rotated in place (vLLM rotary semantics), and the rotated
        key and the value go into the Q8_0 cache at layer_slot_mapping."""
        kp, vp = q8_planes(kv_cache, self.num_kv_heads, self.head_size)
        n = layer_slot_mapping.shape[0]
        D = self.head_size
        q = query[:n].view(n, self.num_heads, D)
        k = key[:n].view(n, self.num_kv_heads, D)
        v = value[:n].view(n, self.num_kv_heads, D)
        pos = positions[:n] if positions.dtype == torch.int64 else positions[:n].to(torch.int64)
        sm = layer_slot_mapping if layer_slot_mapping.dtype == torch.int64 else layer_slot_mapping.to(torch.int64)
        gfx906_fa.rope_and_cache_q8_kv(pos, q, k, v, cos_sin_cache, is_neox, sm, kp, vp)

    @classmethod
    def bound_bytes(cls, heads, limits: tuple[int, int, int]) -> int:
        """The workspace every batch within the scheduler limits needs, plus
        the tile-image room up to image_room_bytes()."""
        max_seqs, max_tokens, max_len = limits
        return workspace_upper_bound(max_seqs, max_tokens, heads, max_len, image_room_bytes())

    @classmethod
    def reserve_workspace(cls, nbytes: int, device: torch.device) -> torch.Tensor:
        """Grow the shared workspace to at least nbytes (never shrinks; grows
        by at least a quarter, so few buffers are ever replaced)."""
        ws = cls._workspace
        if ws is None or ws.numel() < nbytes or ws.device != device:
            if device.type == "cuda" and torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    f"GFX906_FA: attention workspace of {nbytes} bytes needed inside graph "
                    "capture; reserve it before capturing (Gfx906FAImpl.reserve_workspace)")
            size = nbytes
            if ws is not None and ws.device == device:
                size = max(nbytes, ws.numel() + ws.numel() // 4)
            if ws is not None and not cls._captured:
                cls._workspace = ws = None  # free it before the larger one is made
            new = gfx906_fa.new_workspace(size, device)
            if ws is not None:
                cls._retired.append(ws)
            cls._workspace = new
        return cls._workspace

    @classmethod
    def _get_workspace(cls, nbytes: int, device: torch.device) -> torch.Tensor:
        return cls.reserve_workspace(nbytes, device)

    def do_kv_cache_update(self, layer: AttentionLayer, key: torch.Tensor, value: torch.Tensor,
                           kv_cache: torch.Tensor, slot_mapping: torch.Tensor):
        """Quantize K and V of the new tokens to Q8_0 and write them at
        slot_mapping (< 0 skips) - one launch (reference lines 405-442)."""
        kp, vp = q8_planes(kv_cache, self.num_kv_heads, self.head_size)
        n = slot_mapping.shape[0]
        sm = slot_mapping if slot_mapping.dtype == torch.int64 else slot_mapping.to(torch.int64)
        gfx906_fa.reshape_and_cache_q8_kv(key[:n], value[:n], sm, kp, vp)

    def forward(self, layer: torch.nn.Module, query: torch.Tensor, key: torch.Tensor,
                value: torch.Tensor, kv_cache: torch.Tensor, attn_metadata: Gfx906FAMetadata,
                output: torch.Tensor | None = None, output_scale: torch.Tensor | None = None,
                output_block_scale: torch.Tensor | None = None) -> torch.Tensor:
        assert output is not None, "Output tensor must be provided."
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("GFX906_FA: output quantization is not supported")
        if attn_metadata is None:
            # Profiling run: reserve the workspace bound here, so that vLLM's
            # memory profile (which sizes the KV cache) counts it.
            if self._limits is not None and query is not None and query.device.type == "cuda":
                heads = set(self._layer_heads) | {(self.num_heads, self.num_kv_heads)}
                self.reserve_workspace(self.bound_bytes(heads, self._limits), query.device)
            return output.fill_(0)
        assert not attn_metadata.use_cascade, "GFX906_FA: cascade is not supported"
        n = attn_metadata.num_actual_tokens
        kp, vp = q8_planes(kv_cache, self.num_kv_heads, self.head_size)
        md = attn_metadata
        B = md.seq_lens.shape[0]
        if torch.cuda.is_current_stream_capturing():
            Gfx906FAImpl._captured = True
        # the regions the call needs; tile images use whatever room the
        # reserved workspace has past them
        ws = self._get_workspace(
            gfx906_fa.plan_info(B, n, self.num_heads, self.num_kv_heads, md.max_query_len,
                                md.max_seq_len, self.head_size)["img_offset"], query.device)
        out = output[:n].view(n, self.num_heads, self.head_size)
        forward_paged(query[:n], kp, vp, md.block_table, md.seq_lens, md.query_start_loc,
                      md.max_query_len, md.max_seq_len, self.scale, out=out, workspace=ws)
        return output


# -----------------------------------------------------------------------------
# Registration (reference lines 536-553)
# -----------------------------------------------------------------------------
def register() -> None:
    """Register Gfx906FABackend as AttentionBackendEnum.CUSTOM."""
    from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend

    register_backend(AttentionBackendEnum.CUSTOM, f"{__name__}.Gfx906FABackend")
    logger.info("GFX906_FA backend registered as AttentionBackendEnum.CUSTOM")


register()
