class VllmConfig:
    """Opaque configuration object (stub)."""
