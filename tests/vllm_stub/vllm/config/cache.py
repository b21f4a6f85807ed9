from typing import Literal

CacheDType = Literal["auto", "float16", "half", "bfloat16", "fp8", "fp8_e4m3", "fp8_e5m2"]
