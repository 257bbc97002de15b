"""Helpers shared by the tests: numpy <-> torch bf16 transfer and the parity checks."""
import numpy as np


def to_dev(a: np.ndarray, dev, kind: str = "bf16"):
    import torch
    a = np.ascontiguousarray(a)
    if kind == "bf16":
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(dev)
    return torch.from_numpy(a).to(dev)


def bf16_bits(t) -> np.ndarray:
    import torch
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def bf16_f32(t) -> np.ndarray:
    return (bf16_bits(t).astype(np.uint32) << 16).view(np.float32)


def rel_errors(got: np.ndarray, ref: np.ndarray):
    """(normwise max|e| / max|ref|, worst elementwise |e| / (|ref| + rms(ref)))."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    e = np.abs(got - ref)
    mx = float(np.max(np.abs(ref))) if ref.size else 0.0
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    norm = float(e.max() / mx) if mx > 0 else float(e.max() if e.size else 0.0)
    elem = float(np.max(e / (np.abs(ref) + rms))) if (ref.size and rms > 0) else norm
    return norm, elem


def assert_parity(got, ref, what: str, tol: float = 1e-2):
    """bf16 tolerance used for every GEMM output and gradient (max rel err
    <= 1e-2 against the f64/f32 oracle): normwise max|e|/max|ref| <= tol and elementwise
    |e| <= tol * (|ref| + rms(ref))."""
    norm, elem = rel_errors(got, ref)
    print(f"[parity] {what}: normwise {norm:.3e} elementwise {elem:.3e} (tol {tol:g})")
    assert np.all(np.isfinite(np.asarray(got, np.float64))), f"{what}: non-finite output"
    assert norm <= tol, f"{what}: normwise rel err {norm:.3e} > {tol}"
    assert elem <= tol, f"{what}: elementwise rel err {elem:.3e} > {tol}"
    return norm, elem
