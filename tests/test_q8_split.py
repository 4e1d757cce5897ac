"""The q8_0 chunked-prefill kernel stages each dequantized value q * d
(q an int8 in [-127, 127], d a q8_0 block's fp16 scale) as two fp16 values,
hi = fp16(q * d) and lo = fma(q, d, -hi) rounded to fp16, and feeds both to
the MFMAs.  That is exact only if lo is representable in fp16 for every
q and every finite scale that keeps |q * d| inside the fp16 range.  Checked
exhaustively here: all 255 q values x all 63,488 finite fp16 scales."""
import numpy as np


def test_hi_lo_split_is_exact_for_every_q8_0_value():
    d = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    d = d[np.isfinite(d)].astype(np.float64)
    q = np.arange(-127, 128, dtype=np.float64)
    exact = q[:, None] * d[None, :]          # exact in float64 (<= 19 significant bits)
    inside = np.abs(exact) < 65520.0         # rounds to a finite fp16
    with np.errstate(over="ignore"):
        hi = exact.astype(np.float16).astype(np.float64)   # one rounding (RNE)
    lo = exact - hi                          # what the fused multiply-add leaves
    with np.errstate(over="ignore", invalid="ignore"):
        lo16 = lo.astype(np.float16).astype(np.float64)
    assert np.array_equal(lo16[inside], lo[inside])
    assert np.array_equal((hi + lo16)[inside], exact[inside])
    # the range limit is real: the largest scale with q = 127 leaves fp16
    assert not inside.all()
