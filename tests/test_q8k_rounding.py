"""The matvec prologue rounds is * x half away from zero (Rust's f32::round,
lib.rs:1797) as trunc(p + copysign(0.5 - 2^-25, p)) with one f32 addition.
This checks that identity for every f32 p with 0.25 <= |p| < 128 (below 0.25
both give 0; the quantisation never produces |p| above 127 (1 + 2^-23)).
CPU only."""
import numpy as np


def test_round_half_away_identity_exhaustive():
    c = np.float32(0.5) - np.float32(2.0 ** -25)
    assert c == np.float32(0.49999997)
    bad = 0
    for e in range(-2, 7):                      # binades [2^e, 2^(e+1)), 0.25 .. 128
        bits = np.uint32((e + 127) << 23) + np.arange(1 << 23, dtype=np.uint32)
        for sign in (1.0, -1.0):
            p = bits.view(np.float32) * np.float32(sign)
            fast = np.trunc((p + np.copysign(c, p)).astype(np.float32))
            ref = np.trunc(p.astype(np.float64) + np.copysign(0.5, p.astype(np.float64)))
            bad += int(np.count_nonzero(fast != ref))
    assert bad == 0
