from typing import NamedTuple


class DeviceCapability(NamedTuple):
    major: int
    minor: int

    def to_int(self) -> int:
        return self.major * 10 + self.minor
