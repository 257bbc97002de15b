"""CPU checks of the pack kernel's arithmetic (reels_amd/csrc/pack.hip), restated in numpy
float32 and compared with the oracle: it must reproduce quantize_frozen_matrix
(src/layers/quantization.jl:35-44) bit for bit.
- the division shortcut (quantize_one): t = w * fl(1/s), exact IEEE division only within 2^-12
  of a half-integer or for non-normal scales;
- the fast path (Elem<T>::mag / absmax, quantize_chunk_fast): magnitude-bit absmax, med3 clamp,
  magic-number rounding whose low byte is the code, per-chunk redo near ties."""
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


# ---- the kernel's fast path, restated in numpy (pack.hip Elem<T>::mag / absmax,
# quantize_chunk_fast): magnitude-bit absmax, c = med3(w * inv, -127, 127), u = c + 1.5 * 2^23
# (float32 add, round to nearest even) whose low byte is the code, and a per-chunk redo with the
# IEEE division when some |c - (u - 1.5 * 2^23)| > 0.5 - 2^-12.
MAGIC = F32(12582912.0)


def fastpath_pack(w, kind):
    """w: float32 array (kind "f32") or uint16 bf16 bits (kind "bf16"); rows of whole chunks."""
    if kind == "bf16":
        bits = np.ascontiguousarray(w, np.uint16)
        mag = (bits & np.uint16(0x7FFF)).max(axis=1).astype(np.uint32) << np.uint32(16)
        wf = (bits.astype(np.uint32) << np.uint32(16)).view(F32)
        E = 8
    else:
        wf = np.ascontiguousarray(w, F32)
        mag = (wf.view(np.uint32) & np.uint32(0x7FFFFFFF)).max(axis=1)
        E = 4
    N, K = wf.shape
    with np.errstate(all="ignore"):
        m = np.where(mag > np.uint32(0x7F800000), F32(np.nan), mag.view(F32)).astype(F32)
        s = (m / F32(127)).astype(F32)
        s[m == 0] = F32(1)
        fast = (s >= F32(2.0 ** -126)) & (s <= F32(3.4028234663852886e38))
        inv = np.where(fast, (F32(1) / s).astype(F32), F32(0)).astype(F32)
        c = np.clip((wf * inv[:, None]).astype(F32), F32(-127), F32(127))
        u = (c + MAGIC).astype(F32)
        e = np.abs((c - (u - MAGIC).astype(F32)).astype(F32))
        redo_chunk = (e.reshape(N, K // E, E) > F32(0.5 - 2.0 ** -12)).any(axis=2)
        redo = np.repeat(redo_chunk, E, axis=1) | ~fast[:, None]
        q = (u.view(np.uint32) & np.uint32(0xFF)).astype(np.uint8).view(np.int8)
        exact_t = (wf / s[:, None]).astype(F32)
        rd = np.rint(np.clip(exact_t, F32(-127), F32(127)))
    bad = redo & ~np.isfinite(rd)
    q = np.where(redo, np.where(bad, 0, np.nan_to_num(rd)).astype(np.int8), q)
    return q, s, int(bad.any())


def _agree_fast(w, kind):
    q1, s1, st1 = fastpath_pack(w, kind)
    q2, s2, st2 = oracle.pack(w, kind)
    assert st1 == st2
    assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32))
    assert np.array_equal(q1, q2), np.argwhere(q1 != q2)[:5]


def test_magic_rounding_low_byte():
    # every integer and half-integer in [-127, 127]: the low byte of fl(c + 1.5 * 2^23) is the
    # two's complement of rint(c), ties to even
    c = np.arange(-254, 255, dtype=np.float64) / 2
    u = (c.astype(F32) + MAGIC).astype(F32)
    low = (u.view(np.uint32) & np.uint32(0xFF)).astype(np.uint8).view(np.int8)
    assert np.array_equal(low, np.rint(c).astype(np.int8))
    # the wrong constant (2^23) breaks negative codes: the check above would catch it
    u2 = (c.astype(F32) + F32(2.0 ** 23)).astype(F32)
    assert not np.array_equal((u2.view(np.uint32) & np.uint32(0xFF)).astype(np.uint8).view(np.int8),
                              np.rint(c).astype(np.int8))


def test_fastpath_matches_reference_random_bf16_and_f32():
    _agree_fast(oracle.normal_bf16(15, (1024, 4096), 0.02, outlier_rate=1e-3), "bf16")
    _agree_fast(oracle.normal_f32(16, (512, 4096), 1.0), "f32")


def test_fastpath_near_ties_and_boundaries():
    rng = np.random.default_rng(17)
    rows = []
    for _ in range(2048):
        absmax = F32(rng.uniform(1e-6, 100.0))
        s = F32(absmax / F32(127))
        k = rng.integers(-127, 127, size=127).astype(np.float64)
        d = rng.choice([0.0, 1e-7, -1e-7, 5e-7, -5e-7, 2e-6, -2e-6, 3e-5, -3e-5], size=127)
        vals = np.clip(((k + 0.5 + d) * np.float64(s)).astype(F32), -absmax, absmax)
        rows.append(np.concatenate([[absmax], vals]).astype(F32))
    w = np.stack(rows)
    _agree_fast(w, "f32")
    _agree_fast(oracle.f32_to_bf16(w), "bf16")
    # scales on both sides of the normal boundary 2^-126, +-127 s exactly, Inf and NaN rows
    tiny = F32(2.0 ** -126) * F32(127)
    b = np.array([[tiny, -tiny / 2, tiny / 3, 0.0],
                  [np.nextafter(tiny, F32(0)), tiny / 2, -tiny / 5, 0.0],
                  [127.0, -127.0, 126.5, -126.5],
                  [np.inf, 1.0, -2.0, 0.5],
                  [np.nan, 1.0, -2.0, 0.5],
                  [3e38, -3e38, 1.0, 0.0]], F32)
    _agree_fast(b, "f32")
