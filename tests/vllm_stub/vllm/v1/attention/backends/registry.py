import enum
import importlib

_OVERRIDES: dict = {}


class AttentionBackendEnum(enum.Enum):
    FLASH_ATTN = "vllm.v1.attention.backends.flash_attn.FlashAttentionBackend"
    TRITON_ATTN = "vllm.v1.attention.backends.triton_attn.TritonAttentionBackend"
    CUSTOM = ""

    def get_path(self) -> str:
        return _OVERRIDES.get(self, self.value)

    def get_class(self):
        path = self.get_path()
        if not path:
            raise ValueError(f"{self.name} has no registered class")
        mod, _, cls = path.rpartition(".")
        return getattr(importlib.import_module(mod), cls)


def register_backend(backend: AttentionBackendEnum, class_path: str) -> None:
    _OVERRIDES[backend] = class_path
