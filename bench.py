"""Benchmark of the Q8_0 paged-attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 200] [--no-cpu] [--no-prefill]
    python bench.py --workload {cfg3,cfg4,cfg5,cfg5-48,cfg5-k6}   (one other configuration)

Headline (``value``): batched decode, cfg2 of the benchmark definition - 32 sequences with
contexts U[2048, 16384], 48 query / 8 KV heads, head_dim 128, fp16 Q, Q8_0
K and V, block_size 16, permuted block tables.  One step = quantize-write the
32 new tokens' K/V into the paged cache + one attention pass over the batch
(one call: the decode kernel writes the new tokens it streams), all inputs
resident in HBM.  ``value`` is the algorithmic HBM bytes of a step
(Q8 K+V of every cached token, Q, O, block-table entries, the new tokens'
K/V in and Q8 out) divided by the measured step time, in GB/s.

Also reported on the same JSON line:
  roofline      - attention pass (decode + split combine) algorithmic bytes /
                  its average duration from HIP events on the launch stream,
                  against 8 TB/s; ``traffic`` from the committed rocprofv3
                  FETCH_SIZE/WRITE_SIZE measurement when present;
                  ``read_ceiling_gbs`` the library's read-only streaming
                  kernel over 2 GiB on the same GPU and
                  ``frac_of_read_ceiling`` the attention rate against it;
                  ``copy_gbs`` a plain 1 GiB device copy (read + write bytes /
                  time), for comparison.
  prefill       - cfg3 (32K causal prefill, bf16, 48/8): attention TFLOP/s
                  (4*D*Hq*sum of visible keys) vs 2.5 PFLOP/s dense fp16/bf16
                  MFMA peak, ``mfma_busy`` (the MFMA-busy fraction of the
                  kernel's SIMD-cycles from the committed rocprofv3 PMC
                  summary), the K/V quantize-write GB/s, and the fused
                  rotary + K/V write GB/s (vs 8 TB/s) over the same tokens,
                  for the bf16 model and again for an fp16 one.
  configs       - the benchmark definition's other configurations, one timed
                  pass set each (the rows --workload prints in full): cfg4
                  (fraction of the summed MFMA + HBM roofline time, with its
                  prefill and decode parts timed alone), cfg5 at 6/1 and at
                  48/8, and the 6-token n-gram verify step at 6/1 (GB/s).
  next_rows     - graph capture: the cfg2 step and a 32 x 32-token decode
                  batch per call, eager vs replayed from a HIP graph; the
                  output epilogue: the reference's fp32 BSHD -> BHSD ->
                  model-dtype copies timed at cfg3's output size (here the
                  kernels write the model dtype in place); prefix chunks:
                  short prefills on long cached prefixes (their row tiles
                  split over the keys), per pass; reference_matrix: the
                  reference benchmark's own decode and prefill shapes through
                  the contiguous forward (and the decode ones through
                  paged_attention).
  cpu_baseline  - the reference's PyTorch CPU path (oracle/cpu_baseline.py)
                  on the host cores this process may use (its affinity mask,
                  capped by OMP_NUM_THREADS; the count is in ``cores``):
                  ``decode`` (also the top-level value) - paged gather +
                  dequantize + fp32 SDPA on whole cfg2 sequences, repeated for
                  a ~10 s budget, same GB/s accounting; ``prefill`` - cfg3's
                  32K prompt q-chunked (dequantize + fp32 SDPA with the causal
                  mask) over kv-head 0's query heads for a ~10 s budget,
                  TFLOP/s of visible keys.

--workload times the attention pass of another configuration of the benchmark
definition instead (the line's roofline is that workload's dominant kernel):
  cfg3     32K causal prefill (MFMA-bound: TFLOP/s)
  cfg4     mixed chunked prefill + decode; the prefill chunks and the decode
           sequences are also timed as batches of their own (``parts``)
  cfg5     speculative verify, 6/1 heads (HBM-bound: GB/s); cfg5-48: 48/8 heads;
           cfg5-k6: 6 verify tokens (the reference's n-gram k=5), 36 rows
  fwd-dec128k  the contiguous forward's decode (B = 1, 8/4, 131072 keys)
  prefix72     8 x (32768 + 12) at 48/8 on 128-row prefill tiles
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "gfx906-fa-vllm_amd")
for _p in (PKG, ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0
PREWARM_PASSES = 600   # cfg2 attention passes before any timing (~65 ms of device work)


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _profile_value(name: str, key: str):
    """A figure from a committed rocprofv3 PMC summary (profiles/<name>.json),
    or None."""
    p = os.path.join(ROOT, "profiles", f"{name}.json")
    if os.path.exists(p):
        try:
            with open(p) as f:
                return json.load(f).get(key)
        except (OSError, ValueError):
            return None
    return None


def _traffic(kernel_tag: str):
    """HBM bytes per launch from a committed rocprofv3 PMC summary, or None."""
    return _profile_value(f"{kernel_tag}_traffic", "hbm_bytes_per_launch")


def timed(fn, steps: int, warmup: int):
    """Average ms of fn() over `steps` calls, from HIP events recorded on the
    stream the kernels are launched on (the library launches on torch's
    current stream), after `warmup` untimed calls."""
    import torch
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record(stream)
    for _ in range(steps):
        fn()
    e.record(stream)
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def timed_warm(fn, steps: int, warmup: int, min_warm_ms: float = 50.0):
    """timed() with at least ``min_warm_ms`` of device work as warm-up:
    back-to-back passes run up to 7 % slower over the first ~10-20 ms after
    set-up (and after a new batch was written), so a handful of warm-up
    passes is not enough for short ones."""
    est = timed(fn, 1, 1)
    return timed(fn, steps, max(warmup, int(min_warm_ms / max(est, 1e-3)) + 1))


def graph_timed(fn, calls: int = 20, replays: int = 10):
    """Average ms of fn() replayed from a HIP graph that captures `calls`
    back-to-back calls (the host launch cost of the eager loop removed)."""
    import torch
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(calls):
            fn()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(replays):
        g.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / (replays * calls)


def graph_replay_times(args, step, dev) -> dict:
    """Per-call time of the cfg2 step and of a small decode batch (32
    sequences of 32 tokens, 48/8), eager vs replayed from a HIP graph."""
    import torch
    import gfx906_fa
    import gfx906_fa_workloads as W
    sb = W.build_batch([32] * 32, [1] * 32, 48, 8, seed=5, device=dev)
    skp, svp = sb.planes()
    sout = torch.empty((sb.num_tokens, sb.Hq, sb.D), dtype=torch.float16, device=dev)
    sws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(
        sb.num_seqs, sb.num_tokens, sb.Hq, sb.Hkv, sb.max_query_len, sb.max_seq_len), dev)

    def small():
        gfx906_fa.paged_attention(sb.query, skp, svp, sb.block_table, sb.seq_lens_t, sb.qsl_t,
                                  sb.max_query_len, sb.max_seq_len, sb.scale, out=sout, workspace=sws)

    return {
        "cfg2_step_us": {"eager": round(timed(step, args.steps, args.warmup) * 1e3, 2),
                         "graph": round(graph_timed(step) * 1e3, 2)},
        "small_decode_us": {"workload": "32 seqs x 32 tokens, 48/8",
                            "eager": round(timed(small, 200, 50) * 1e3, 2),
                            "graph": round(graph_timed(small) * 1e3, 2)},
    }


def output_epilogue_ms(dev) -> dict:
    """The reference's output epilogue - fp32 BSHD result transposed to BHSD,
    then copied into the model-dtype output (extension/gfx906_fa.cpp:264,
    extension/gfx906_fa_backend.py:527-528) - timed at cfg3's output size.
    The kernels here write the model dtype in place: no epilogue."""
    import torch
    T3, H3 = 32768, 48
    o32 = torch.empty((1, T3, H3, 128), dtype=torch.float32, device=dev)
    o16 = torch.empty((T3, H3 * 128), dtype=torch.bfloat16, device=dev)

    def ref_epilogue():
        bhsd = o32.transpose(1, 2).contiguous()
        o16.copy_(bhsd.transpose(1, 2).reshape(T3, H3 * 128))

    o32.normal_()
    ms = timed(ref_epilogue, 10, 3)
    del o32, o16
    torch.cuda.empty_cache()
    return {"workload": "cfg3 output, 32768 x 48 x 128", "reference_epilogue_ms": round(ms, 4), "here_ms": 0.0}


def prefix_chunk_times(dev) -> dict:
    """Short prefills on long cached prefixes (prefix caching), 48/8, fp16
    out: one attention pass each.  The prefill plan splits their row tiles
    over the keys; TFLOP/s counts the visible keys of the real rows only."""
    import torch
    import gfx906_fa
    import gfx906_fa_workloads as W
    res = {"workload": "48/8, fp16 out, paged Q8 cache"}
    for name, B, ctx, nq in (("1x(65536+50)", 1, 65536, 50), ("8x(32768+12)", 8, 32768, 12),
                             ("1x(129024+2048)", 1, 129024, 2048)):
        b = W.build_batch([ctx + nq] * B, [nq] * B, 48, 8, seed=7, device=dev, host_values=False)
        o = torch.empty((b.num_tokens, b.Hq, b.D), dtype=torch.float16, device=dev)
        ws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(
            b.num_seqs, b.num_tokens, b.Hq, b.Hkv, b.max_query_len, b.max_seq_len), dev)
        ms = timed(_attn_fn(b, o, ws), 10, 3)
        res[name] = {"us": round(ms * 1e3, 1), "tflops": round(b.flops() / (ms * 1e-3) / 1e12, 1),
                     "cache_gbs": round(b.kv_bytes() / (ms * 1e-3) / 1e9, 1)}
        del b, o, ws
        torch.cuda.empty_cache()
    return res


# The reference's own benchmark matrix (tests/bench.py:39-66 of the
# reference): gfx906_fa.forward(q fp32, AoS Q8_0 K, fp16 V, scale) at batch 1,
# no mask, non-causal.
REF_DECODE = [("dec_128", 8, 4, 128), ("dec_512", 8, 4, 512), ("dec_1k", 8, 4, 1024), ("dec_4k", 8, 4, 4096),
              ("dec_8k", 8, 4, 8192), ("dec_16k", 8, 4, 16384), ("dec_32k", 8, 4, 32768),
              ("dec_64k", 8, 4, 65536), ("dec_94k", 8, 4, 94208), ("dec_128k", 8, 4, 131072),
              ("mmx_dec_1k", 48, 8, 1024), ("mmx_dec_8k", 48, 8, 8192), ("mmx_dec_32k", 48, 8, 32768),
              ("mmx_dec_94k", 48, 8, 94208)]
REF_PREFILL = [("pre_512", 8, 4, 512), ("pre_1k", 8, 4, 1024), ("pre_2k", 8, 4, 2048), ("pre_4k", 8, 4, 4096),
               ("pre_8k", 8, 4, 8192)]


def reference_matrix(dev) -> dict:
    """The reference benchmark's shapes through the contiguous ``forward``
    (device time per call from HIP events: the call's kernels and its q / out
    transposes, not the host launch cost), and each decode shape also through
    ``paged_attention`` on a Q8_0 paged cache (block_size 16, permuted table).
    Decode GB/s counts the bytes each path must read and write: forward the
    AoS K (136 B) and fp16 V (256 B) per key and kv-head, paged the Q8 K and
    V (272 B); prefill TFLOP/s counts 4 * D * Hq * Sq * Skv (non-causal)."""
    import torch
    import gfx906_fa
    import gfx906_fa_workloads as W
    res = {"workload": "B = 1, D = 128, fp32 q, scale 1/sqrt(128); forward: AoS Q8_0 K + fp16 V, no mask; "
                       "paged: Q8_0 K + V pages, fp16 q and out"}
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    for name, hq, hkv, skv in REF_DECODE:
        q = torch.randn((1, hq, 1, 128), generator=g, device=dev)
        k = torch.randn((1, hkv, skv, 128), generator=g, device=dev).mul_(0.1).half()
        v = torch.randn((1, hkv, skv, 128), generator=g, device=dev).mul_(0.1).half()
        kq = gfx906_fa.quantize_q8_0(k)
        del k
        ms = timed(lambda: gfx906_fa.forward(q, kq, v, 1.0 / 128 ** 0.5), 50, 10)
        fbytes = hkv * skv * (136 + 256) + 2 * hq * 128 * 4
        b = W.build_batch([skv], [1], hq, hkv, seed=1, device=dev, host_values=False)
        o = torch.empty((1, hq, 128), dtype=torch.float16, device=dev)
        ws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(1, 1, hq, hkv, 1, skv), dev)
        ms_p = timed(_attn_fn(b, o, ws), 50, 10)
        res[name] = {"heads": f"{hq}/{hkv}", "skv": skv, "forward_us": round(ms * 1e3, 1),
                     "forward_gbs": round(fbytes / (ms * 1e-3) / 1e9, 1), "paged_us": round(ms_p * 1e3, 1),
                     "paged_gbs": round(b.hbm_bytes(2) / (ms_p * 1e-3) / 1e9, 1)}
        del q, kq, v, b, o, ws
        torch.cuda.empty_cache()
    for name, hq, hkv, sq in REF_PREFILL:
        q = torch.randn((1, hq, sq, 128), generator=g, device=dev)
        k = torch.randn((1, hkv, sq, 128), generator=g, device=dev).mul_(0.1).half()
        v = torch.randn((1, hkv, sq, 128), generator=g, device=dev).mul_(0.1).half()
        kq = gfx906_fa.quantize_q8_0(k)
        ms = timed(lambda: gfx906_fa.forward(q, kq, v, 1.0 / 128 ** 0.5), 20, 5)
        fl = 4.0 * 128 * hq * sq * sq
        res[name] = {"heads": f"{hq}/{hkv}", "sq": sq, "skv": sq, "forward_us": round(ms * 1e3, 1),
                     "forward_tflops": round(fl / (ms * 1e-3) / 1e12, 2)}
        del q, k, kq, v
        torch.cuda.empty_cache()
    return res


def gather_rates(dev) -> dict:
    """The standalone gathers at cfg2's shape (32 sequences, contexts
    U[2048, 16384], 8 kv-heads, block_size 16, permuted block tables, Sk the
    longest context rounded up to 32): the reference's contract (AoS Q8_0 K
    rows + fp16 V rows -> contiguous [B, Hkv, Sk, row],
    extension/gfx906_fa_gather.cu:190-357) and the planar Q8 K+V planes ->
    AoS Q8_0 rows.  Algorithmic bytes: the valid rows read, the K rows of
    valid tokens and every V row (zeroed past seq_len) written, the block
    table read."""
    import numpy as np
    import torch
    import gfx906_fa
    import gfx906_fa_workloads as W
    sl, _, _, Hkv, _ = W.cfg_shape("cfg2")
    sl = np.asarray(sl, np.int32)
    B, bs = len(sl), 16
    rng = np.random.default_rng(3)
    bt, nb = W.make_block_table(rng, sl, bs)
    Sk = (int(sl.max()) + 31) // 32 * 32
    M = bt.shape[1]
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    kc = torch.randint(0, 256, (nb, bs, Hkv, 136), dtype=torch.uint8, device=dev, generator=g)
    vc = torch.randn((nb, bs, Hkv, 128), dtype=torch.float16, device=dev, generator=g)
    btt = torch.from_numpy(bt).to(dev)
    slt = torch.from_numpy(sl).to(dev)
    ko = torch.empty((B, Hkv, Sk, 136), dtype=torch.uint8, device=dev)
    vo = torch.empty((B, Hkv, Sk, 128), dtype=torch.float16, device=dev)
    valid = int(np.minimum(sl, Sk).astype(np.int64).sum())
    ref_bytes = valid * Hkv * (136 + 256) + valid * Hkv * 136 + B * Hkv * Sk * 256 + B * M * 4
    ms_ref = timed(lambda: gfx906_fa.gather_paged_kv_q8(kc, vc, btt, slt, Sk, k_out=ko, v_out=vo), 20, 5)
    del kc, vc
    cache = torch.randint(0, 256, (nb, 2, Hkv, bs // 16 * 2176), dtype=torch.uint8, device=dev, generator=g)
    vq = torch.empty((B, Hkv, Sk, 136), dtype=torch.uint8, device=dev)
    pl_bytes = valid * Hkv * 272 + valid * Hkv * 136 + B * Hkv * Sk * 136 + B * M * 4
    ms_pl = timed(lambda: gfx906_fa.gather_paged_kv_q8q8(cache[:, 0], cache[:, 1], btt, slt, Sk,
                                                          k_out=ko, v_out=vq), 20, 5)
    del cache, ko, vo, vq
    torch.cuda.empty_cache()
    gbs = lambda n, ms: round(n / (ms * 1e-3) / 1e9, 1)  # noqa: E731
    return {"workload": f"cfg2 shape: {B} seqs, {valid} tokens, {Hkv} kv-heads, Sk {Sk}",
            "reference_contract": {"us": round(ms_ref * 1e3, 1), "bytes": ref_bytes, "gbs": gbs(ref_bytes, ms_ref),
                                   "frac_of_hbm_peak": round(ref_bytes / (ms_ref * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
            "planar_to_aos_q8": {"us": round(ms_pl * 1e3, 1), "bytes": pl_bytes, "gbs": gbs(pl_bytes, ms_pl),
                                 "frac_of_hbm_peak": round(pl_bytes / (ms_pl * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}}


def _attn_fn(b, out, ws):
    import gfx906_fa
    kp, vp = b.planes()

    def f():
        gfx906_fa.paged_attention(b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t,
                                  b.max_query_len, b.max_seq_len, b.scale, out=out, workspace=ws)
    return f


def extra_workload(wl: str, dev, steps: int, warmup: int) -> dict:
    """The rows after the hot path as workloads of their own (for kernel
    traces and counters of their kernels):
      fwd-dec128k  the contiguous forward, B = 1 decode, 8/4 heads, 131072
                   keys (AoS Q8_0 K + fp16 V; flat_decode_kernel + merge)
      prefix72     8 x (32768 + 12) at 48/8: 72 rows per kv-head on 128-row
                   prefill tiles, split over the keys"""
    import torch
    import gfx906_fa
    import gfx906_fa_workloads as W
    base = {"metric": "Q8 paged decode HBM GB/s (% of peak); causal prefill attn TFLOP/s @32K", "n_gpus": 1,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "data": "synthetic"}
    if wl == "fwd-dec128k":
        g = torch.Generator(device=dev)
        g.manual_seed(0)
        hq, hkv, skv = 8, 4, 131072
        q = torch.randn((1, hq, 1, 128), generator=g, device=dev)
        k = torch.randn((1, hkv, skv, 128), generator=g, device=dev).mul_(0.1).half()
        v = torch.randn((1, hkv, skv, 128), generator=g, device=dev).mul_(0.1).half()
        kq = gfx906_fa.quantize_q8_0(k)
        del k
        ms = timed_warm(lambda: gfx906_fa.forward(q, kq, v, 1.0 / 128 ** 0.5), steps, warmup)
        nbytes = hkv * skv * (136 + 256) + 2 * hq * 128 * 4
        gbs = nbytes / (ms * 1e-3) / 1e9
        return dict(base, steps=steps, ms_per_step=round(ms, 5), dtype="f32 q, Q8_0 K, f16 V",
                    value=round(gbs, 1), unit="GB/s",
                    config={"workload": "fwd-dec128k: gfx906_fa.forward, B = 1, 8/4 heads, Sq 1, Skv 131072, "
                                        "AoS Q8_0 K + fp16 V (the reference benchmark's dec_128k)",
                            "algorithmic_bytes": nbytes, "parallelism": "single GPU"},
                    roofline={"bound": "hbm", "kernel": "flat_decode_kernel+flat_combine_kernel",
                              "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                              "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": _traffic("flat_decode_fwd128k"),
                              "avg_us": round(ms * 1e3, 2)})
    b = W.build_batch([32768 + 12] * 8, [12] * 8, 48, 8, seed=7, device=dev, host_values=False)
    o = torch.empty((b.num_tokens, b.Hq, b.D), dtype=torch.float16, device=dev)
    ws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(
        b.num_seqs, b.num_tokens, b.Hq, b.Hkv, b.max_query_len, b.max_seq_len), dev)
    ms = timed_warm(_attn_fn(b, o, ws), steps, warmup)
    hb = b.hbm_bytes(out_bytes_per_elem=2)
    gbs = hb / (ms * 1e-3) / 1e9
    return dict(base, steps=steps, ms_per_step=round(ms, 5), dtype="f16", value=round(gbs, 1), unit="GB/s",
                config={"workload": "prefix72: 8 x (32768 cached + 12 new tokens), 48/8 heads, fp16, Q8_0 K+V "
                                    "(72 rows per kv-head: 128-row prefill tiles, split over the keys)",
                        "algorithmic_bytes": hb, "flop": b.flops(), "parallelism": "single GPU",
                        "pf_rows": gfx906_fa.plan_info(b.num_seqs, b.num_tokens, b.Hq, b.Hkv, b.max_query_len,
                                                       b.max_seq_len)["pf_rows"]},
                roofline={"bound": "hbm", "kernel": "attn_prefill_kernel (128-row tiles)+attn_prefill_combine_kernel",
                          "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": _traffic("attn_prefill_prefix72"),
                          "avg_us": round(ms * 1e3, 2)})


def workload_result(wl: str, dev, steps: int, warmup: int) -> dict:
    """One attention pass of cfg3 / cfg4 / cfg5 (inputs resident in HBM),
    timed with HIP events on the launch stream: the full JSON line of
    ``--workload wl``."""
    import torch

    import gfx906_fa
    import gfx906_fa_workloads as W

    if wl in ("fwd-dec128k", "prefix72"):
        return extra_workload(wl, dev, steps, warmup)

    name = {"cfg5-48": "cfg5", "cfg5-k6": "cfg5k6"}.get(wl, wl)
    verify = name in ("cfg5", "cfg5k6")
    heads = (48, 8) if wl == "cfg5-48" else None
    b = W.build_cfg(name, device=dev, heads=heads)
    odt = torch.bfloat16 if b.dtype == "bf16" else torch.float16

    def new_out(bb):
        return torch.empty((bb.num_tokens, bb.Hq, bb.D), dtype=odt, device=dev)

    def new_ws(bb):
        return gfx906_fa.new_workspace(gfx906_fa.workspace_size(
            bb.num_seqs, bb.num_tokens, bb.Hq, bb.Hkv, bb.max_query_len, bb.max_seq_len), dev)

    steps = steps if verify else max(3, min(10, steps // 5))
    # warm-up: the given steps, and at least ~50 ms of device work
    ms = timed_warm(_attn_fn(b, new_out(b), new_ws(b)), steps, max(2, warmup if verify else 2))
    fl, hb = b.flops(), b.hbm_bytes(out_bytes_per_elem=2)
    gbs, tfs = hb / (ms * 1e-3) / 1e9, fl / (ms * 1e-3) / 1e12
    res = {
        "metric": "Q8 paged decode HBM GB/s (% of peak); causal prefill attn TFLOP/s @32K",
        "n_gpus": 1, "steps": steps, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": b.dtype, "data": "synthetic",
        "config": {"workload": f"{wl}: {W.CONFIGS[name]}", "num_seqs": b.num_seqs,
                   "num_tokens": b.num_tokens, "heads": f"{b.Hq}/{b.Hkv}", "total_context": int(b.seq_lens.sum()),
                   "algorithmic_bytes": hb, "flop": fl, "parallelism": "single GPU"},
    }
    if verify:
        res.update({"value": round(gbs, 1), "unit": "GB/s"})
        res["roofline"] = {"bound": "hbm", "kernel": "attn_decode_kernel+attn_combine_kernel",
                           "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "avg_us": round(ms * 1e3, 2)}
    elif name == "cfg3":
        res.update({"value": round(tfs, 2), "unit": "TFLOP/s"})
        res["roofline"] = {"bound": "mfma", "kernel": "attn_prefill_kernel", "achieved": round(tfs, 2),
                           "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tfs / MFMA_PEAK_TFLOPS, 4),
                           "traffic": None, "avg_us": round(ms * 1e3, 2),
                           "mfma_busy": _profile_value("attn_prefill_cfg3_mfma", "mfma_busy_frac")}
    else:  # cfg4: both bounds; the parts timed as batches of their own
        npf = int((b.q_lens > 1).sum())
        pf, dc = W.sub_batch(b, 0, npf), W.sub_batch(b, npf, b.num_seqs)
        ms_pf = timed_warm(_attn_fn(pf, new_out(pf), new_ws(pf)), steps, 2)
        ms_dc = timed_warm(_attn_fn(dc, new_out(dc), new_ws(dc)), max(steps, 20), 40)
        t_roof = pf.flops() / (MFMA_PEAK_TFLOPS * 1e12) + dc.hbm_bytes(2) / (HBM_PEAK_GBS * 1e9)
        res.update({"value": round(t_roof / (ms * 1e-3), 4), "unit": "fraction of the summed roofline time"})
        res["roofline"] = {"bound": "mfma+hbm", "kernel": "attn_prefill_kernel+attn_decode_kernel",
                           "achieved": round(t_roof * 1e3, 4), "peak": round(ms, 4), "unit": "ms (roofline / measured)",
                           "frac": round(t_roof / (ms * 1e-3), 4), "traffic": None}
        res["parts"] = {
            "prefill_chunks": {"ms": round(ms_pf, 4), "flop": pf.flops(),
                               "tflops": round(pf.flops() / (ms_pf * 1e-3) / 1e12, 2),
                               "frac_of_mfma_peak": round(pf.flops() / (ms_pf * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4)},
            "decode_seqs": {"ms": round(ms_dc, 4), "bytes": dc.hbm_bytes(2),
                            "gbs": round(dc.hbm_bytes(2) / (ms_dc * 1e-3) / 1e9, 1),
                            "frac_of_hbm_peak": round(dc.hbm_bytes(2) / (ms_dc * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        }
    del b
    torch.cuda.empty_cache()
    return res


def config_rows(dev, steps: int, warmup: int) -> dict:
    """The benchmark definition's other configurations, one timed pass set
    each, for the default line: cfg4 (mixed chunked prefill + decode: the
    fraction of the summed MFMA + HBM roofline time), cfg5 at 6/1 (5 verify
    tokens, the tensor-parallel shard) and 48/8, and the reference's n-gram
    verify step (6 tokens, k = 5) at 6/1 (HBM GB/s against 8 TB/s)."""
    rows = {}
    for wl in ("cfg4", "cfg5", "cfg5-48", "cfg5-k6"):
        r = workload_result(wl, dev, steps, warmup)
        e = {"workload": r["config"]["workload"], "heads": r["config"]["heads"], "passes": r["steps"],
             "ms": r["ms_per_step"], "value": r["value"], "unit": r["unit"], "frac": r["roofline"]["frac"]}
        if "parts" in r:
            e["summed_roofline_ms"] = r["roofline"]["achieved"]
            e["parts"] = r["parts"]
        else:
            e["bytes"] = r["config"]["algorithmic_bytes"]
        rows[wl] = e
    return rows


def calib_copy(dev, mib: int) -> int:
    """A plain device copy of known size (the run's last dispatch): its
    FETCH_SIZE / WRITE_SIZE readings scale the other kernels' counters to
    bytes."""
    import torch
    n = mib << 20
    src = torch.empty(n // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    return n


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # The first ~10 ms of back-to-back steps after set-up run up to 7 % slower
    # (measured 115 -> 110 -> 108 us per cfg2 step over successive 60-step
    # loops), so the default warm-up covers ~20 ms of steps.
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the cfg4 / cfg5 rows of the default line")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="also run one plain device copy of this size (rocprof counter calibration)")
    ap.add_argument("--workload", default="cfg2",
                    choices=["cfg2", "cfg3", "cfg4", "cfg5", "cfg5-48", "cfg5-k6", "fwd-dec128k", "prefix72"])
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(attention shards by KV head with no exchange inside the kernel)", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import gfx906_fa
    import gfx906_fa_workloads as W

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload != "cfg2":
        res = workload_result(args.workload, dev, args.steps, args.warmup)
        if args.calib_copy_mib:
            res["calib_copy_bytes"] = calib_copy(dev, args.calib_copy_mib)
        print(json.dumps(res), flush=True)
        return 0

    # ---------------- cfg2 decode -----------------------------------------
    b = W.build_cfg("cfg2", device=dev)
    kp, vp = b.planes()
    B = b.num_seqs
    # the step's new tokens: the last position of every sequence
    last = torch.from_numpy(np.cumsum(b.seq_lens.astype(np.int64)) - 1).to(dev)
    k_new = b.key.index_select(0, last).contiguous()
    v_new = b.value.index_select(0, last).contiguous()
    s_new = b.slot_mapping.index_select(0, last).contiguous()
    out = torch.empty((b.num_tokens, b.Hq, b.D), dtype=torch.float16, device=dev)
    ws_bytes = gfx906_fa.workspace_size(B, b.num_tokens, b.Hq, b.Hkv, b.max_query_len, b.max_seq_len)
    ws = gfx906_fa.new_workspace(ws_bytes, dev)

    def attn():
        gfx906_fa.paged_attention(b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t,
                                  b.max_query_len, b.max_seq_len, b.scale, out=out, workspace=ws)

    def step():
        # the step's cache write folded into the attention launch (the
        # backend's decode step); the same bytes and output as the write
        # kernel followed by attn()
        gfx906_fa.paged_attention(b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t,
                                  b.max_query_len, b.max_seq_len, b.scale, out=out, workspace=ws,
                                  new_key=k_new, new_value=v_new, slot_mapping=s_new)

    # Pre-warm.  Back-to-back passes run up to 7 % slower over the first
    # ~10-20 ms of device work after set-up (successive 60-step loops of the
    # cfg2 step measured 115, 110 and 108 us), and the driver's --warmup is a
    # handful of steps.  So the ceiling measurements and PREWARM_PASSES
    # attention passes run first; their device time is reported as
    # ``prewarm_ms``, apart from the --warmup steps.  The ceilings: the
    # library's read-only streaming kernel over 2 GiB (the bound for a pass
    # that reads ~1000x what it writes), and a plain 1 GiB device copy (read
    # + write bytes over its time, reported for comparison).
    stream = torch.cuda.current_stream()
    csrc = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    cdst = torch.empty_like(csrc)
    rsrc = torch.ones(1 << 29, dtype=torch.float32, device=dev)
    rwords = torch.empty(gfx906_fa.lib().gfx906_fa_amd_stream_read_words(), dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    pw0, pw1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    pw0.record(stream)
    ms_copy = timed(lambda: cdst.copy_(csrc), 20, 5)
    copy_gbs = 2 * csrc.numel() * 4 / (ms_copy * 1e-3) / 1e9
    ms_read = timed(lambda: gfx906_fa.stream_read(rsrc, rwords), 20, 5)
    read_gbs = rsrc.numel() * 4 / (ms_read * 1e-3) / 1e9
    for _ in range(PREWARM_PASSES):
        attn()
    pw1.record(stream)
    torch.cuda.synchronize()
    prewarm_ms = pw0.elapsed_time(pw1)
    del csrc, cdst, rsrc, rwords

    # the headline: exactly --steps steps after --warmup steps
    ms_step = timed(step, args.steps, args.warmup)
    # the attention pass alone (roofline): at least 50 timed passes
    attn_calls = max(args.steps, 50)
    ms_attn = timed(attn, attn_calls, args.warmup)

    step_bytes = b.hbm_bytes(out_bytes_per_elem=2) + B * b.Hkv * (2 * 2 * 128 + 2 * 136) + B * 8
    attn_bytes = b.hbm_bytes(out_bytes_per_elem=2)
    value = step_bytes / (ms_step * 1e-3) / 1e9
    achieved = attn_bytes / (ms_attn * 1e-3) / 1e9
    traffic = _traffic("attn_decode_cfg2")

    res = {
        "metric": "Q8 paged decode HBM GB/s (% of peak); causal prefill attn TFLOP/s @32K",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": "cfg2 batched decode: 32 seqs, ctx U[2048,16384] (seeded), 48/8 heads, "
                        "head_dim 128, fp16 Q, Q8_0 K+V, block_size 16, permuted block tables",
            "num_seqs": B, "total_context": int(b.seq_lens.sum()), "kv_q8_bytes": b.kv_bytes(),
            "step_bytes": step_bytes, "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm", "kernel": "attn_decode_kernel+attn_combine_kernel",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic, "algorithmic_bytes": attn_bytes, "avg_us": round(ms_attn * 1e3, 2),
            "read_ceiling_gbs": round(read_gbs, 1), "frac_of_read_ceiling": round(achieved / read_gbs, 4),
            "copy_gbs": round(copy_gbs, 1), "timed_passes": attn_calls,
        },
        "prewarm_ms": round(prewarm_ms, 2),
        "prewarm": f"before timing: a 1 GiB device copy x 25, a 2 GiB read-only stream x 25 and "
                   f"{PREWARM_PASSES} attention passes ({prewarm_ms:.1f} ms of device work), then the "
                   f"{args.warmup} --warmup steps",
    }

    # ---------------- the rows after the hot path -------------------------
    # graph capture (not in the counter calibration runs, which profile the
    # eager kernels only)
    graph = None if args.calib_copy_mib else graph_replay_times(args, step, dev)

    # ---------------- cfg3 prefill (secondary) ------------------------------
    cpu_prefill = None
    if not args.no_prefill:
        del b, out, ws
        torch.cuda.empty_cache()
        p = W.build_cfg("cfg3", device=dev)
        pk, pv = p.planes()
        pout = torch.empty((p.num_tokens, p.Hq, p.D), dtype=torch.bfloat16, device=dev)
        pws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(
            p.num_seqs, p.num_tokens, p.Hq, p.Hkv, p.max_query_len, p.max_seq_len), dev)

        def pattn():
            gfx906_fa.paged_attention(p.query, pk, pv, p.block_table, p.seq_lens_t, p.qsl_t,
                                      p.max_query_len, p.max_seq_len, p.scale, out=pout, workspace=pws)

        def pwrite():
            gfx906_fa.reshape_and_cache_q8_kv(p.key, p.value, p.slot_mapping, pk, pv)

        # fused rotary embedding + K/V quantize-write (the backend's
        # do_rope_and_kv_cache_update) over the same 32768 tokens; it rotates
        # query and key in place, so it runs after the attention timing
        T3 = p.key.shape[0]
        pos3 = torch.arange(T3, dtype=torch.int64, device=dev)
        cs3 = W.rope_cos_sin_cache(T3, p.D, torch.bfloat16, dev)

        def prope():
            gfx906_fa.rope_and_cache_q8_kv(pos3, p.query, p.key, p.value, cs3, True, p.slot_mapping, pk, pv)

        psteps = max(3, min(10, args.steps // 5))
        ms_p = timed(pattn, psteps, 2)
        ms_w = timed(pwrite, psteps, 2)
        ms_r = timed(prope, psteps, 2)
        # the same write for an fp16 model (its own kernel instantiation)
        q16, k16, v16 = p.query.half(), p.key.half(), p.value.half()
        cs16 = W.rope_cos_sin_cache(T3, p.D, torch.float16, dev)

        def prope16():
            gfx906_fa.rope_and_cache_q8_kv(pos3, q16, k16, v16, cs16, True, p.slot_mapping, pk, pv)

        ms_r16 = timed(prope16, psteps, 2)
        del q16, k16, v16
        rbytes = W.rope_write_bytes(T3, p.Hq, p.Hkv, p.D)
        fl = p.flops()
        wbytes = p.key.numel() * 2 * 2 + p.key.shape[0] * p.Hkv * 2 * 136 + p.key.shape[0] * 8
        res["prefill"] = {
            "workload": "cfg3: 1 x 32768 causal prefill from the paged Q8 cache, 48/8, bf16",
            "attn_ms": round(ms_p, 4), "tflops": round(fl / (ms_p * 1e-3) / 1e12, 2),
            "mfma_peak_tflops": MFMA_PEAK_TFLOPS,
            "frac": round(fl / (ms_p * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4), "flop": fl,
            "mfma_busy": _profile_value("attn_prefill_cfg3_mfma", "mfma_busy_frac"),
            "kv_write_ms": round(ms_w, 4), "kv_write_gbs": round(wbytes / (ms_w * 1e-3) / 1e9, 1),
            "rope_kv_write_ms": round(ms_r, 4), "rope_kv_write_bytes": rbytes,
            "rope_kv_write_gbs": round(rbytes / (ms_r * 1e-3) / 1e9, 1),
            "rope_kv_write_frac": round(rbytes / (ms_r * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "rope_kv_write_f16_ms": round(ms_r16, 4),
            "rope_kv_write_f16_gbs": round(rbytes / (ms_r16 * 1e-3) / 1e9, 1),
        }
        if not args.no_cpu:
            # the reference's CPU path on the same prompt, q-chunked, kv-head
            # by kv-head for a time budget (attention is linear in heads, so
            # the TFLOP/s over the heads run is the rate of all 48)
            from oracle import cpu_baseline as CB
            pcache = p.kv_cache.cpu().numpy()
            pk_aos, pv_aos = CB.aos_from_planar(pcache)
            del pcache
            q3 = p.query.float().cpu().contiguous()
            secs, pflop, pheads, pdone, pnch, g3, pthr = CB.time_cpu_prefill(
                q3, pk_aos, pv_aos, p.block_table_np[0], int(p.seq_lens[0]), p.scale, chunk=1024,
                budget_s=args.cpu_budget)
            cpu_prefill = {
                "value": round(pflop / secs / 1e12, 4), "unit": "TFLOP/s", "cores": pthr, "kind": "port",
                "sample": f"cfg3 32K causal prefill, q-chunked (1024 query rows per fp32 SDPA with the causal "
                          f"mask), kv-head by kv-head: {pdone} chunks = {pdone / pnch:.2f} of the {p.Hkv} "
                          f"kv-heads' {g3} query heads each (attention is linear in heads), dequantize "
                          f"included; {pflop:.3e} FLOP of visible keys in {secs:.2f} s",
                "est_full_cfg3_s": round(fl / (pflop / secs), 1),
            }
            del pk_aos, pv_aos, q3
        del p, pout
        torch.cuda.empty_cache()

    # ---------------- the other configurations ---------------------------
    if not args.no_configs and not args.calib_copy_mib:
        res["configs"] = config_rows(dev, args.steps, args.warmup)

    if graph is not None:
        res["next_rows"] = {"graph_replay": graph,
                            "output_epilogue": output_epilogue_ms(dev),
                            "prefix_chunks": prefix_chunk_times(dev),
                            "gather": gather_rates(dev),
                            "reference_matrix": reference_matrix(dev)}

    if args.calib_copy_mib:
        res["calib_copy_bytes"] = calib_copy(dev, args.calib_copy_mib)

    # ---------------- CPU baseline -----------------------------------------
    if not args.no_cpu:
        from oracle import cpu_baseline as CB
        b = W.build_cfg("cfg2", device=dev)
        cache = b.kv_cache.cpu().numpy()
        q = b.query.float().cpu()
        k_aos, v_aos = CB.aos_from_planar(cache)
        secs, tokens, nseq, passes, thr = CB.time_cpu_decode(
            q, k_aos, v_aos, b.block_table_np, b.seq_lens, b.q_lens, b.scale, budget_s=args.cpu_budget)
        sub_bytes = tokens * b.Hkv * 2 * 136 + nseq * b.Hq * b.D * 4
        dec = {
            "value": round(sub_bytes / secs / 1e9, 3), "unit": "GB/s", "cores": thr, "kind": "port",
            "sample": f"{nseq} cfg2 sequence decodes ({passes} whole passes over the 32, then the rest in "
                      f"batch order; {tokens} cached tokens read): paged gather + dequantize + fp32 SDPA, "
                      f"{secs:.2f} s",
        }
        res["cpu_baseline"] = dict(dec, cpu=_cpu_model(), decode=dec)
        if cpu_prefill is not None:
            res["cpu_baseline"]["prefill"] = cpu_prefill
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
