import contextlib


class VllmConfig:
    """Opaque configuration object (stub)."""


_current = None


def get_current_vllm_config():
    """The configuration set around model construction (stub: a default
    VllmConfig when none is set, as vLLM does)."""
    return _current if _current is not None else VllmConfig()


@contextlib.contextmanager
def set_current_vllm_config(cfg):
    global _current
    prev, _current = _current, cfg
    try:
        yield
    finally:
        _current = prev
