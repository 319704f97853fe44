"""``TriMulPrecision``, the enum cuequivariance_torch uses for trimul's precision argument
(same members and values as the reference shim's _trimul_precision.py:9-14)."""

import enum


class TriMulPrecision(enum.IntEnum):
    NONE = -1
    DEFAULT = 0
    TF32 = 1
    TF32x3 = 2
    IEEE = 3
