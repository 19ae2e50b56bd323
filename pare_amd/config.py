"""The subset of Pare's QuantDtype / QuantConfig that the INT4 linear path reads.

Mirrors pare/core/dtype.py:9-97 and pare/config.py:44-100 for the fields the
forward path uses (bits, dtype, scheme, granularity, group_size, sym,
act_order). Calibration, AWQ, SmoothQuant and sensitivity fields are not read
by the forward path and are not carried. A reference ``QuantConfig`` object can
be passed anywhere this one is accepted (duck typing on the same attributes).
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum


@dataclass(frozen=True)
class _DTypeSpec:
    bits: int
    is_float: bool
    signed: bool


class QuantDtype(Enum):
    """Names and ranges of pare/core/dtype.py:44-50."""

    INT2 = _DTypeSpec(2, False, False)
    INT3 = _DTypeSpec(3, False, False)
    INT4 = _DTypeSpec(4, False, False)
    INT8 = _DTypeSpec(8, False, True)
    FP8_E4M3 = _DTypeSpec(8, True, True)
    FP8_E5M2 = _DTypeSpec(8, True, True)
    NF4 = _DTypeSpec(4, True, True)

    @property
    def bits(self) -> int:
        return self.value.bits

    @property
    def is_float(self) -> bool:
        return self.value.is_float

    def _code_range(self) -> tuple[int, int]:
        if self.value.is_float:
            raise TypeError(f"{self.name} is a floating-point format: it has no integer code range")
        n = self.bits
        return (-(1 << (n - 1)), (1 << (n - 1)) - 1) if self.value.signed else (0, (1 << n) - 1)

    @property
    def qmin(self) -> int:
        return self._code_range()[0]

    @property
    def qmax(self) -> int:
        return self._code_range()[1]

    @classmethod
    def from_bits(cls, bits: int, *, signed: bool = False) -> "QuantDtype":
        """The integer format of `bits` bits: INT8 (signed) for 8 whatever
        `signed` says; the 2-, 3- and 4-bit formats exist unsigned only."""
        if bits == 8:
            return cls.INT8
        if not signed:
            for member in (cls.INT2, cls.INT3, cls.INT4):
                if member.bits == bits:
                    return member
        raise ValueError(f"QuantDtype.from_bits: no integer format with bits={bits}, signed={signed}")


@dataclass
class QuantConfig:
    bits: int = 4
    dtype: QuantDtype | None = None
    scheme: str = "rtn"
    granularity: str = "per_group"
    group_size: int = 128
    sym: bool = False
    damp_percent: float = 0.01
    act_order: bool = False

    _SCHEMES = ("rtn", "gptq", "awq", "smoothquant")
    _GRANULARITIES = ("per_tensor", "per_channel", "per_group")

    def __post_init__(self) -> None:
        checks = (("scheme", self.scheme, self._SCHEMES),
                  ("granularity", self.granularity, self._GRANULARITIES),
                  ("bits", self.bits, (2, 3, 4, 8)))
        for field, value, allowed in checks:
            if value not in allowed:
                raise ValueError(f"QuantConfig.{field}={value!r} is not one of {allowed}")
        if self.dtype is None:
            self.dtype = QuantDtype.from_bits(self.bits)

    @property
    def effective_dtype(self) -> QuantDtype:
        assert self.dtype is not None
        return self.dtype


def is_int4(config) -> bool:
    """True for an INT4 config of either this package or the reference."""
    dt = getattr(config, "effective_dtype", None)
    return getattr(dt, "name", None) == "INT4"


def kernel_group_size(config, in_features: int) -> int:
    """Group size the kernel path uses (pare/layers/linear.py:145)."""
    return config.group_size if config.granularity == "per_group" else in_features
