"""CPU: bench.py's command-line contract that needs no GPU."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    """One GPU only: --gpus above 1 exits 2 with a message that says so, before
    any GPU work (the run ends before torch is imported)."""
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_bench_help_lists_workloads():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--help"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 0
    for w in ("cfg3", "cfg4", "cfg5", "cfg5-48", "--steps", "--warmup"):
        assert w in r.stdout


def test_bench_reads_the_committed_pmc_figures():
    """The bench line's ``traffic`` (decode) and ``mfma_busy`` (prefill) come
    from the committed rocprofv3 summaries under profiles/."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    t = m._traffic("attn_decode_cfg2")
    assert isinstance(t, int) and t > 600_000_000
    busy = m._profile_value("attn_prefill_cfg3_mfma", "mfma_busy_frac")
    assert 0.0 < busy < 1.0
    assert m._profile_value("no_such_profile", "x") is None
