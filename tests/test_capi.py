"""CPU: the C-ABI library loads and exports every entry point the header
declares; argument validation fails before any GPU work (no compute calls)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gfx906_fa_amd.h")
LIB = os.path.join(ROOT, "gfx906-fa-vllm_amd", "libgfx906_fa_amd.so")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"^\s*#.*$", "", src, flags=re.M)     # preprocessor lines (macros are not symbols)
    return sorted(set(re.findall(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\(", src)) -
                  {"extern", "if", "defined"})


def test_header_declares_expected_entry_points():
    names = _declared()
    for n in ["launch_quantize_q8_0_dense", "launch_reshape_and_cache_q8",
              "launch_gather_paged_kv_q8", "gfx906_fa_amd_cache_write_kv",
              "gfx906_fa_amd_paged_attention", "gfx906_fa_amd_paged_attention_workspace_size",
              "gfx906_fa_amd_gather_planar", "gfx906_fa_amd_gather_rows",
              "gfx906_fa_amd_paged_attention_workspace_bound", "gfx906_fa_amd_paged_attention_plan_info",
              "gfx906_fa_amd_device_cus", "gfx906_fa_amd_paged_attention_noalloc"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "build the library first (__graft_entry__.build())"
    lib = ctypes.CDLL(LIB)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_validation_errors_without_gpu():
    import gfx906_fa  # loads the library; no GPU needed
    L = gfx906_fa.lib()
    assert b"gfx950" in L.gfx906_fa_amd_version()
    # head_size 64 is rejected before any launch (hipErrorInvalidValue = 1)
    err = L.gfx906_fa_amd_paged_attention(None, 1, 0, 0, None, None, 0, 0, None, 0, None, None,
                                          None, 1, 1, 1, 8, 1, 64, 16, 1, 16, 0.1, None, 1, 0, 0,
                                          None, 0, None)
    assert err == 1
    # block size not a multiple of 16
    err = L.gfx906_fa_amd_paged_attention(None, 1, 0, 0, None, None, 0, 0, None, 0, None, None,
                                          None, 1, 1, 1, 8, 1, 128, 24, 1, 16, 0.1, None, 1, 0, 0,
                                          None, 0, None)
    assert err == 1
    # quantize: D not a multiple of 32
    assert L.gfx906_fa_amd_quantize_q8_0(None, 1, None, 4, 48, None) == 1
    # planar write: head size must be 128
    assert L.gfx906_fa_amd_cache_write_kv(None, None, 1, None, None, None, 1, 1, 64, 16,
                                          0, 0, 0, 0, 0, 0, None) == 1
    # empty work is a no-op success (returns before any HIP call)
    assert L.gfx906_fa_amd_quantize_q8_0(None, 1, None, 0, 128, None) == 0
    assert L.gfx906_fa_amd_cache_write_kv(None, None, 1, None, None, None, 0, 8, 128, 16,
                                          0, 0, 0, 0, 0, 0, None) == 0
    assert L.gfx906_fa_amd_paged_attention(None, 1, 0, 0, None, None, 0, 0, None, 0, None, None,
                                           None, 1, 0, 0, 48, 8, 128, 16, 1, 16, 0.1, None, 1, 0, 0,
                                           None, 0, None) == 0
    assert L.gfx906_fa_amd_gather_planar(None, None, None, None, None, None, 0, 8, 32, 128, 16, 4,
                                         0, 0, None) == 0
    # fused rotary + write: rot_dim 72 is not a multiple of 16 (neox); fp32 rows;
    # a valid configuration with no tokens is a no-op
    rope = L.gfx906_fa_amd_rope_cache_write_kv
    args = [None, None, None, 1, None, None, 1, 128, 4096, 128, 1, None, None, None, 0, 8, 2, 128, 16,
            0, 0, 0, 0, 0, 0, 0, 0, None]
    assert rope(*args) == 0
    bad = list(args)
    bad[9] = 72
    assert rope(*bad) == 1
    bad = list(args)
    bad[3] = 0
    assert rope(*bad) == 1
    # attention with the write folded in: key / value / slot_mapping are required
    err = L.gfx906_fa_amd_paged_attention_kv_write(None, 1, 0, 0, None, None, 0, 0, None, 0, None, None,
                                                   None, 1, 1, 1, 8, 1, 128, 16, 1, 16, 0.1, None, 1, 0,
                                                   0, None, 0, None, None, 1, 0, 0, 0, 0, None, None)
    assert err == 1
    # streaming-read helper: a byte count that is not a multiple of 16, or too
    # few output words, is refused before any launch; zero bytes is a no-op
    nw = L.gfx906_fa_amd_stream_read_words()
    assert nw > 0
    assert L.gfx906_fa_amd_stream_read(None, 0, None, 0, None) == 0
    assert L.gfx906_fa_amd_stream_read(None, 24, None, nw, None) == 1
    assert L.gfx906_fa_amd_stream_read(None, 32, None, nw - 1, None) == 1
    # allocation-free attention: a batch whose plan exceeds the library's
    # scratch is refused on the host, before the scratch is looked up or any
    # work is enqueued (no device needed)
    f = L.gfx906_fa_amd_paged_attention_noalloc
    big_b = 40_000_000  # per-sequence prefix sums alone exceed 64 MiB
    assert f(None, 1, 0, 0, None, None, 0, 0, None, 0, None, None, None, 1, big_b, big_b, 48, 8, 128,
             16, 1, 16, 0.1, None, 1, 0, 0, None) == 1
    # contiguous decode: more than 16 rows per kv-head (2 queries x 16 q-heads
    # per kv-head) and misaligned K are refused before any launch; no work is
    # a no-op
    fd = L.gfx906_fa_amd_flat_decode
    assert fd(None, 0, 0, 0, None, None, None, None, 1, 2, 16, 1, 100, 128, 0.1, None, 0, 0, None, 0,
              None) == 1
    assert fd(None, 0, 0, 0, ctypes.c_void_p(8), ctypes.c_void_p(16), ctypes.c_void_p(16), None, 1, 1, 8, 4, 100,
              128, 0.1, None, 0, 0, None, 0, None) == 1
    assert fd(None, 0, 0, 0, None, None, None, None, 1, 1, 8, 4, 0, 128, 0.1, None, 0, 0, None, 0, None) == 0
    assert L.gfx906_fa_amd_flat_decode_workspace_size(1, 1, 8, 4, 128) == 256
    # the scratch copy helper refuses ranges past the scratch
    assert L.gfx906_fa_amd_noalloc_scratch_copy(None, 0, 16, None) == 1
    assert L.gfx906_fa_amd_noalloc_scratch_copy(ctypes.c_void_p(16), 64 << 20, 16, None) == 1


def test_workspace_size_plan():
    import gfx906_fa
    # stream-K decode always needs the plan + two partial slots per workgroup
    a = gfx906_fa.workspace_size(1, 1, 8, 1, 1, 1024)
    b = gfx906_fa.workspace_size(32, 32, 48, 8, 1, 16384)
    assert a > 0 and a % 256 == 0 and b % 256 == 0
    assert b >= a  # the per-sequence prefix grows with num_seqs
    # 30 verify rows (6 q-heads x 5 tokens) use 32-row slots: twice the partials
    assert gfx906_fa.workspace_size(8, 40, 6, 1, 5, 131077) > gfx906_fa.workspace_size(8, 8, 6, 1, 1, 131077)
    # independent of the context length (stream-K shares work per wave)
    assert gfx906_fa.workspace_size(32, 32, 48, 8, 1, 1 << 20) == b
    # a prefill launch also holds the partials of split row tiles: 3 ceil(CUs / Hkv)
    # slots per kv head of 256 rows x (128 + 2) floats.  The CU count is the
    # library's own query (the device's count on a GPU host; without a device
    # the library plans for 256, the MI355X count, which this then pins)
    cus = gfx906_fa.device_cus()
    assert cus > 0
    pf = gfx906_fa.workspace_size(1, 50, 48, 8, 50, 65586)
    assert pf >= 3 * (-(-cus // 8)) * 8 * 256 * 130 * 4
    # A launch whose sequences can have 32 row tiles (2048 tokens x 6 q-heads
    # = 48 here) also takes room for its 64-key tiles dequantized once
    # (35840 bytes per tile and kv head, one prefill sequence here), capped
    # at 1 GiB; the regions every call needs do not depend on the context
    # length
    i1 = gfx906_fa.plan_info(1, 2048, 48, 8, 2048, 65586)
    i2 = gfx906_fa.plan_info(1, 2048, 48, 8, 2048, 1 << 20)
    assert i1["img_offset"] == i2["img_offset"] and i1["img_offset"] % 256 == 0
    assert i1["img_bytes"] == -(-(65586 // 64 + 1) * 8 * 35840 // 256) * 256
    assert i2["img_bytes"] == 1 << 30
    assert gfx906_fa.workspace_size(1, 2048, 48, 8, 2048, 65586) == i1["img_offset"] + i1["img_bytes"]
    assert gfx906_fa.workspace_size(1, 2048, 48, 8, 2048, 1 << 20) == i2["img_offset"] + (1 << 30)
    # the 50-token chunk (2 row tiles) and a decode-only shape take none
    assert gfx906_fa.plan_info(1, 50, 48, 8, 50, 65586)["img_bytes"] == 0
    assert pf == gfx906_fa.plan_info(1, 50, 48, 8, 50, 65586)["img_offset"]
    assert gfx906_fa.plan_info(32, 32, 48, 8, 1, 16384)["img_bytes"] == 0
    # the bar: 32 row tiles (8192 rows at one q-head per kv-head) take room,
    # 31 (7936 rows) none
    assert gfx906_fa.plan_info(1, 8192, 8, 8, 8192, 9000)["img_bytes"] > 0
    assert gfx906_fa.plan_info(1, 7936, 8, 8, 7936, 9000)["img_bytes"] == 0
    # kv-head counts that do not divide the CU count round the slots up per head
    for hkv in (3, 5, 7, 12):
        need = 3 * (-(-cus // hkv)) * hkv * 256 * 130 * 4
        assert gfx906_fa.workspace_size(2, 200, 2 * hkv, hkv, 100, 9000) >= need
        info = gfx906_fa.plan_info(2, 200, 2 * hkv, hkv, 100, 9000)
        assert info["pf_slots_max"] == 3 * (-(-cus // hkv)) and info["cus"] == cus
        assert info["bytes"] == gfx906_fa.workspace_size(2, 200, 2 * hkv, hkv, 100, 9000)


def test_plan_info():
    import torch
    import gfx906_fa
    if not torch.cuda.is_available():
        assert gfx906_fa.device_cus() == 256  # the fallback without a device
    d = gfx906_fa.plan_info(32, 32, 48, 8, 1, 16384)   # cfg2 decode: one class, no prefill
    assert (d["decode_classes"], d["dec_rows_max"], d["prefill"], d["pf_header_offset"]) == (1, 16, 0, -1)
    v = gfx906_fa.plan_info(8, 40, 6, 1, 5, 131077)    # 30 verify rows: the 32-row class
    assert (v["decode_classes"], v["dec_rows_max"], v["prefill"]) == (1, 32, 0)
    m = gfx906_fa.plan_info(64, 8252, 48, 8, 2048, 131072)  # mixed: both classes and a work list
    assert (m["decode_classes"], m["dec_rows_max"], m["prefill"]) == (2, 64, 1)
    assert 0 < m["pf_header_offset"] < m["bytes"] and m["pf_header_offset"] % 256 == 0
    assert gfx906_fa.plan_info(1, 32768, 48, 8, 32768, 32768)["decode_classes"] == 0
    # 33-48 rows: the three-row-group class (48-row tiles); 49-64 rows: the
    # two-row-group class in 32-row chunks.  Mixed row counts up to 48 take
    # one class per tile size (16, 32, 48 rows).
    u36 = gfx906_fa.plan_info(8, 48, 6, 1, 6, 131078)        # 6 verify tokens at 6/1: 36 rows
    assert (u36["decode_classes"], u36["dec_rows_max"], u36["prefill"]) == (1, 48, 0)
    u64 = gfx906_fa.plan_info(3, 24, 8, 1, 8, 5000)          # 8 tokens at 8/1: 64 rows
    assert (u64["decode_classes"], u64["dec_rows_max"], u64["prefill"]) == (1, 64, 0)
    mix48 = gfx906_fa.plan_info(4, 18, 6, 1, 6, 30000)       # 5 + 6 + 1 + 6 tokens at 6/1
    assert (mix48["decode_classes"], mix48["dec_rows_max"], mix48["prefill"]) == (3, 48, 0)
    mix64 = gfx906_fa.plan_info(3, 14, 8, 1, 8, 5000)        # 1 + 5 + 8 tokens at 8/1
    assert (mix64["decode_classes"], mix64["dec_rows_max"], mix64["prefill"]) == (2, 64, 0)
    g40 = gfx906_fa.plan_info(3, 5, 40, 1, 3, 5000)          # G = 40, 1 + 1 + 3 tokens: 40 and 120 rows
    assert (g40["decode_classes"], g40["dec_rows_max"], g40["prefill"]) == (1, 64, 1)
    assert mix48["bytes"] <= gfx906_fa.workspace_bound(4, 18, 6, 1)
    # below 8 sub-pages per decode workgroup 33-48 rows stay in 32-row chunks
    s36 = gfx906_fa.plan_info(8, 48, 6, 1, 6, 2006)          # 8 x (2000 + 6) at 6/1
    assert (s36["decode_classes"], s36["dec_rows_max"], s36["prefill"]) == (1, 64, 0)
    smix = gfx906_fa.plan_info(4, 18, 6, 1, 6, 3000)
    assert (smix["decode_classes"], smix["dec_rows_max"], smix["prefill"]) == (2, 64, 0)
    # prefill tile rows: 128-row key-interleaved tiles up to 128 rows per
    # kv-head (the longest sequence's), 256-row tiles above
    assert d["pf_rows"] == 0 and m["pf_rows"] == 256
    for q, G, want in ((11, 6, 128), (12, 6, 128), (16, 8, 128), (128, 1, 128), (129, 1, 256), (32, 6, 256),
                       (51, 5, 256), (50, 6, 256), (48, 8, 256), (32768, 6, 256)):
        info = gfx906_fa.plan_info(1, q, 8 * G, 8, q, 65536)
        assert info["pf_rows"] == want, (q, G, info["pf_rows"])
    assert g40["pf_rows"] == 128                              # 120 rows beside decode rows
    pc = gfx906_fa.plan_info(33, 12 + 32, 48, 8, 12, 32768)   # 32 decodes + a 12-token chunk
    assert (pc["decode_classes"], pc["dec_rows_max"], pc["pf_rows"]) == (2, 64, 128)
    with pytest.raises(RuntimeError):
        gfx906_fa.plan_info(1, 1, 6, 4, 1, 1)             # heads not divisible


def test_ops_reject_cpu_tensors():
    import torch
    import gfx906_fa
    with pytest.raises(RuntimeError, match="CUDA/HIP"):
        gfx906_fa.quantize_q8_0(torch.zeros(4, 32, dtype=torch.float16))


def test_noalloc_scratch_size_stated():
    """The allocation-free entry point's scratch is stated in the header."""
    src = open(HEADER).read()
    m = re.search(r"#define GFX906_FA_AMD_SCRATCH_BYTES \(\(size_t\)(\d+) << (\d+)\)", src)
    assert m and int(m.group(1)) << int(m.group(2)) == 64 << 20
