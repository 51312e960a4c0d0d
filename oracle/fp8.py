"""OCP FP8 E4M3FN written from the format definition (test infrastructure).

E4M3FN: 1 sign bit, 4 exponent bits (bias 7), 3 mantissa bits, no
infinities, a single NaN pattern per sign (exponent and mantissa all ones),
largest finite value 448.  gfx950 MFMA and conversion instructions use this
format (reference evidence: lib/Dialect/FlyROCDL/CDNA4/MmaAtom.cpp:164,
kernels/qk_norm_rope_quant.py:78-92), and ``torch.float8_e4m3fn`` is the same
format, which is how the tests pin these functions against a library routine.
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0
E4M3_BIAS = 7


def decode_table() -> np.ndarray:
    """float64 value of each of the 256 byte codes, from the bit fields."""
    out = np.empty(256, dtype=np.float64)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exp = (code >> 3) & 0xF
        man = code & 0x7
        if exp == 0xF and man == 0x7:
            out[code] = np.nan
        elif exp == 0:
            out[code] = sign * man * 2.0 ** (1 - E4M3_BIAS - 3)
        else:
            out[code] = sign * (1.0 + man / 8.0) * 2.0 ** (exp - E4M3_BIAS)
    return out


_TABLE = decode_table()


def decode(codes: np.ndarray) -> np.ndarray:
    """uint8 codes -> float64 values."""
    return _TABLE[np.asarray(codes, dtype=np.uint8)]


def encode(x: np.ndarray) -> np.ndarray:
    """float -> uint8 code, round to nearest, ties to even mantissa.

    Magnitudes that round past 448 become NaN (0x7F / 0xFF), as the
    non-saturating cast of ``torch.Tensor.to(float8_e4m3fn)`` does; NaN and
    infinities map to NaN.  Brute force over the 127 non-negative finite
    codes: pick the nearest, break ties toward the even code.
    """
    x = np.asarray(x, dtype=np.float64)
    finite_vals = _TABLE[:127]  # codes 0x00..0x7E, increasing
    mag = np.abs(x)
    idx = np.searchsorted(finite_vals, mag, side="left")
    idx = np.clip(idx, 1, 126)
    lo = finite_vals[idx - 1]
    hi = finite_vals[idx]
    choose_hi = (mag - lo > hi - mag) | ((mag - lo == hi - mag) & ((idx % 2) == 0))
    code = np.where(choose_hi, idx, idx - 1).astype(np.int64)
    code = np.where(mag <= 0.0, 0, code)
    # Past the largest finite value: ties at 464 go to the even code 0x7E
    # (448); anything larger rounds into the NaN pattern.
    code = np.where(mag > 464.0, 0x7F, code)
    code = np.where(np.isnan(x) | np.isinf(x), 0x7F, code)
    sign = np.where(np.signbit(x), 0x80, 0)
    return (code | sign).astype(np.uint8)
