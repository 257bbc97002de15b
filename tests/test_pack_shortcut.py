"""CPU check of the pack kernel's division shortcut (reels_amd/csrc/pack.hip quantize_one):
t = w * fl(1/s), exact IEEE division only within 2^-12 of a half-integer or for non-normal
scales, must reproduce quantize_frozen_matrix (src/layers/quantization.jl:35-44) bit for bit.
The shortcut is restated in numpy float32 and compared with the oracle."""
import numpy as np

import oracle

F32 = np.float32


def shortcut_pack(w):
    w = np.ascontiguousarray(w, F32)
    with np.errstate(all="ignore"):
        m = np.max(np.abs(w), axis=1)
        s = (m / F32(127)).astype(F32)
        s[m == 0] = F32(1)
        fast = (s >= F32(2.0 ** -126)) & np.isfinite(s)
        inv = np.where(fast, (F32(1) / s).astype(F32), F32(0)).astype(F32)
        t = (w * inv[:, None]).astype(F32)
        near = np.abs(t - np.rint(t)) > F32(0.5 - 2.0 ** -12)
        exact = (w / s[:, None]).astype(F32)
        t = np.where(near | ~fast[:, None], exact, t)
        c = np.where(t > 127, F32(127), np.where(t < -127, F32(-127), t))
        rd = np.rint(c)
    bad = ~np.isfinite(rd)
    return np.where(bad, 0, rd).astype(np.int8), s, int(bad.any())


def _agree(w):
    q1, s1, st1 = shortcut_pack(w)
    q2, s2, st2 = oracle.pack(np.ascontiguousarray(w, F32), "f32")
    assert st1 == st2
    assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32))
    assert np.array_equal(q1, q2), np.argwhere(q1 != q2)[:5]


def test_shortcut_matches_reference_random():
    _agree(oracle.bf16_to_f32(oracle.normal_bf16(5, (2048, 2048), 0.02, outlier_rate=1e-3)))
    _agree(oracle.normal_f32(6, (1024, 4096), 1.0))


def test_shortcut_matches_reference_near_ties():
    rng = np.random.default_rng(9)
    rows = []
    for _ in range(4096):
        absmax = F32(rng.uniform(1e-6, 100.0))
        s = F32(absmax / F32(127))
        k = rng.integers(-126, 126, size=255).astype(np.float64)
        d = rng.choice([0.0, 1e-7, -1e-7, 5e-7, -5e-7, 2e-6, -2e-6, 3e-5, -3e-5], size=255)
        vals = np.clip(((k + 0.5 + d) * np.float64(s)).astype(F32), -absmax, absmax)
        rows.append(np.concatenate([[absmax], vals]).astype(F32))
    _agree(np.stack(rows))


def test_shortcut_special_scales():
    ulp = np.array([1], np.uint32).view(F32)[0]
    w = np.array([[127 * ulp, 64 * ulp, 0, -127 * ulp],
                  [10 * ulp, 5 * ulp, 10 * ulp, 5 * ulp],
                  [0, 0, 0, 0],
                  [3e38, -3e38, 1.0, 0.0],
                  [1e-38, 5e-39, -1e-38, 0.0]], F32)
    _agree(w)
