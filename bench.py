"""Benchmark: int8-weight LoRA linear forward + dX + dA + dB on Wan-2.1-14B block shapes, 1 GPU.

One step = one pass over the six projections of a Wan-2.1-14B transformer block at 32760 tokens
(480x832x81 frames: latent 21x60x104, patch 1x2x2): self-attention q/k/v/o 5120->5120 and the FFN
5120->13824->5120, each an int8 per-output-channel frozen weight (packed from bf16 ~N(0, 0.02))
with a rank-32 LoRA (alpha 32, A and B ~N(0, 0.01)), bf16 activations ~N(0, 1) and output
gradients ~N(0, 1). Forward runs q, k, v, o, ffn.0, ffn.2; backward runs them in reverse, each
producing dX, dA and dB. Inputs are synthetic and already resident in HBM when timing starts.

Prints one JSON line (see the keys below). Per-kernel durations come from HIP events recorded by
the library around every launch on the launch stream, over the timed steps themselves.

    python bench.py [--gpus 1] [--steps 10] [--warmup 3] [--cpu-seconds 15] [--no-pack]

A second workload, reported under "pack": quantize_frozen_matrix on the full 40-layer
Wan-2.1-14B weight set (per layer q, k, v, o 5120x5120, ffn.0 13824x5120, ffn.2 5120x13824: 9.857e9
bf16 elements ~N(0, 0.02) with 0.1% outliers at +-20 sigma), packed as two row-stacked launches
(all K = 5120 rows, then all K = 13824 rows; packing is row-independent).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

METRIC = ("TFLOP/s and % bf16-MFMA peak, int8-W LoRA linear fwd+bwd, Wan-14B shapes, 1 GPU")
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (published)
PEAK_TFLOPS = {"bf16": 2500.0, "f16": 2500.0, "f32": 157.3}  # dense MFMA, published
PEAK_HBM_GBS = 8000.0
TOKENS = 32760
RANK = 32
ALPHA = 32.0
WARM_S = 0.05  # untimed back-to-back calls before timing a call of tens of microseconds
# HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs of this script (KiB per
# dispatch scaled by a 1 GiB device copy: FETCH x 2.0, WRITE x 1.0), averaged over one step's
# launches; the commands and per-kernel figures are in profiles/.
GEMM_TRAFFIC_BYTES = 4663654453
GEMM_TRAFFIC_NOTE = ("mean over one step's 12 GEMM launches (q/k/v/o 3.04 GB, ffn 7.60-8.30 GB); "
                     "FETCH_SIZE includes Infinity Cache hits; algorithmic mean 0.946 GB")
PACK_TRAFFIC_BYTES = 14792000000  # mean of the two launches (21.088 + 8.496 GB), ratio 1.000
PROJECTIONS = [("self_attn.q", 5120, 5120), ("self_attn.k", 5120, 5120),
               ("self_attn.v", 5120, 5120), ("self_attn.o", 5120, 5120),
               ("ffn.0", 5120, 13824), ("ffn.2", 13824, 5120)]


def linear_flops(M, K, N, r):
    return 4.0 * M * N * K + 6.0 * M * r * (K + N)


def gemm_flops(mode, M, K, N, r):
    """Algorithmic flops of one i8gemm launch: the base product plus the fused LoRA term."""
    return 2.0 * M * N * K + 2.0 * M * r * (N if mode == "fwd" else K)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="approximate CPU work for the cpu_baseline sample (0 disables it)")
    ap.add_argument("--tokens", type=int, default=TOKENS)
    ap.add_argument("--offload", choices=("none", "stream", "sync"), default="none",
                    help="cpu_offload: int8 codes and scales in pinned host memory, streamed to the "
                         "GPU one projection ahead of use on a copy stream (stream: WeightStreamer, "
                         "two slots) or copied right before each use (sync: the reference's "
                         "per-call upload)")
    ap.add_argument("--dtype", choices=("bf16", "f16", "f32"), default="bf16",
                    help="activation / LoRA element type: bf16 (the default workload) or f16 "
                         "(the reference's own int8 compute precision, the _f16 entry points)")
    ap.add_argument("--no-pack", action="store_true", help="skip the pack workload")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the config 1 / 2 / 4 / 5a lines")
    ap.add_argument("--no-attention", action="store_true", help="skip the attention workload")
    ap.add_argument("--attention-only", action="store_true",
                    help="run only the attention workload")
    ap.add_argument("--pack-only", action="store_true", help="run only the pack workload")
    ap.add_argument("--configs-only", default=None,
                    help="run only these config lines (comma-separated, e.g. cfg5a) and exit")
    ap.add_argument("--trace", choices=("gemm", "all"), default="gemm",
                    help="kernels bracketed by HIP events inside the timed steps: the GEMMs only "
                         "(their durations give roofline.achieved; the per-kernel breakdown comes "
                         "from one extra untimed step with every kernel traced) or every kernel")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run three 1 GiB device-to-device copies (the reference kernel for "
                         "scaling FETCH_SIZE / WRITE_SIZE counters to bytes) and exit")
    return ap.parse_args()


def vendor_gemm_tflops(dev, M, K, N, seconds=1.5, dtype=None):
    """torch.matmul (hipBLASLt; bf16 unless dtype says otherwise, fp32 without TF32) on one
    Wan-14B projection shape, timed over a
    sustained loop (~seconds, like the timed bench steps: the GPU runs at its power cap, so short
    bursts and sustained loops clock differently): the practical MFMA ceiling for a dense GEMM
    of this size on this GPU, measured in the same run."""
    import torch
    dtype = dtype or torch.bfloat16
    x = torch.randn((M, K), device=dev).to(dtype)
    w = torch.randn((N, K), device=dev).to(dtype)
    for _ in range(3):
        torch.matmul(x, w.t())
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):
        torch.matmul(x, w.t())
    torch.cuda.synchronize()
    reps = max(10, int(seconds / max((time.perf_counter() - t0) / 5, 1e-6)))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        torch.matmul(x, w.t())
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del x, w
    torch.cuda.empty_cache()
    return 2.0 * M * N * K / (ms * 1e-3) / 1e12


PACK_LAYERS = 40
PACK_SETS = [(PACK_LAYERS * (4 * 5120 + 13824), 5120), (PACK_LAYERS * 5120, 13824)]  # (rows, K)


def pack_bench(dev, reps=3):
    """Times the pack kernel on the 40-layer 14B weight set; returns the "pack" result object."""
    import torch
    from reels_amd import _lib
    L = _lib.lib()
    gen = torch.Generator(device=dev).manual_seed(77)
    mats = []
    for rows, K in PACK_SETS:
        w = torch.empty((rows, K), dtype=torch.bfloat16, device=dev)
        step = 16384
        for r0 in range(0, rows, step):
            r1 = min(rows, r0 + step)
            c = torch.randn((r1 - r0, K), generator=gen, device=dev).mul_(0.02)
            u = torch.rand((r1 - r0, K), generator=gen, device=dev)
            sign = torch.where(u < 0.0005, -1.0, 1.0)
            c = torch.where(u < 0.001, sign * 0.4, c)
            w[r0:r1] = c.to(torch.bfloat16)
            del c, u, sign
        q = torch.empty((rows, K), dtype=torch.int8, device=dev)
        sc = torch.empty((rows,), dtype=torch.float32, device=dev)
        mats.append((w, q, sc, rows, K))
    status = torch.zeros((1,), dtype=torch.int32, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())

    def run():
        for (w, q, sc, rows, K) in mats:
            _lib.check("reels_hip_i8_pack", L.reels_hip_i8_pack(p(w), _lib.BF16, rows, K, K, p(q),
                                                                p(sc), p(status), st))
    run()
    torch.cuda.synchronize()
    _lib.check("reels_hip_trace_start", L.reels_hip_trace_start(16 * reps))
    t0 = time.perf_counter()
    for _ in range(reps):
        run()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    recs = [(n, ms) for (n, ms) in _lib.trace_records() if n.startswith("pack_rows")]
    elems = sum(rows * K for (_, _, _, rows, K) in mats)
    nbytes = sum(3 * rows * K + 4 * rows for (_, _, _, rows, K) in mats)
    ms = (t1 - t0) * 1e3 / reps
    kern_ms = sum(ms_ for (_, ms_) in recs) / reps
    gbs = nbytes / (kern_ms * 1e-3) / 1e9
    assert int(status.item()) == 0
    # sampled rows of each timed launch (input and the GPU's codes and scales) for the bit-exact
    # comparison in the CPU-baseline leg
    rng = torch.Generator().manual_seed(5)
    samples = []
    for (w, q, sc, rows, K) in mats:
        idx = torch.cat([torch.randint(0, rows, (62,), generator=rng), torch.tensor([0, rows - 1])])
        ix = idx.to(dev)
        samples.append((w[ix].view(torch.int16).cpu().numpy(), q[ix].cpu().numpy(),
                        sc[ix].cpu().numpy(), rows, K))
    del mats
    torch.cuda.empty_cache()
    copy = copy_gbs(dev)
    out = {"metric": "pack GB/s (bf16 read + int8 codes + f32 scales)", "value": round(gbs, 1),
           "unit": "GB/s", "ms": round(ms, 4), "kernel_ms": round(kern_ms, 4),
           "elements": elems, "bytes": nbytes,
           "roofline": {"kernel": "pack_rows_kernel", "bound": "hbm", "achieved": round(gbs, 1),
                        "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                        "traffic": PACK_TRAFFIC_BYTES,
                        "device_copy": {"what": "torch copy_ of a 4 GiB buffer (read + write bytes), "
                                                "same run", "gbs": round(copy, 1),
                                        "achieved_over_copy": round(gbs / copy, 4)}}}
    return out, samples


# Wan-2.1-14B self-attention of one block: 32760 tokens (the projection workload's token
# count), 40 heads of 128, no mask, not causal (src/models/wan21/transformer.jl:199)
ATT_SHAPE = (1, 32760, 40, 128)


def attention_flops(B, Sq, Sk, H, D):
    """Algorithmic flops of forward (Q K^T and P V: 4 B H Sq Sk D) and backward (2.5 x forward:
    dV, dP, dQ, dK and the score recomputation counted once, the usual accounting)."""
    f = 4.0 * B * H * Sq * Sk * D
    return f, 2.5 * f


def attention_bench(dev, reps=3):
    """Times reels_hip_attention_fwd + _bwd on the Wan-14B self-attention shape; returns the
    "attention" result object, with torch's fused SDPA (flash / memory-efficient backends only)
    on the same shape as the vendor reference."""
    import torch
    from reels_amd import _lib, memory_efficient_attention, memory_efficient_attention_backward
    L = _lib.lib()
    B, S, H, D = ATT_SHAPE
    gen = torch.Generator(device=dev).manual_seed(5)
    q, k, v, dy = (torch.randn((B, S, H, D), generator=gen, device=dev).to(torch.bfloat16)
                   for _ in range(4))

    def step():
        r = memory_efficient_attention(q, k, v)
        memory_efficient_attention_backward(q, k, v, dy, r.cache)
    step()
    torch.cuda.synchronize()
    _lib.check("reels_hip_trace_start", L.reels_hip_trace_start(16 * reps))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    kern = {}
    for n, t in _lib.trace_records():
        c, tot = kern.get(n, (0, 0.0))
        kern[n] = (c + 1, tot + t)
    ff, fb = attention_flops(B, S, S, H, D)
    fwd_ms = kern.get("attn_fwd_kernel", (1, float("nan")))[1] / reps
    bwd_ms = sum(t for n, (c, t) in kern.items() if n != "attn_fwd_kernel") / reps
    tflops = (ff + fb) / (ms * 1e-3) / 1e12
    vendor = None
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        qt, kt, vt, dyt = (x.transpose(1, 2).contiguous() for x in (q, k, v, dy))
        qt.requires_grad_(); kt.requires_grad_(); vt.requires_grad_()
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            def vstep():
                o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt)
                o.backward(dyt)
                qt.grad = kt.grad = vt.grad = None
            vstep()
            torch.cuda.synchronize()
            e0.record()
            for _ in range(reps):
                vstep()
            e1.record()
            torch.cuda.synchronize()
        vms = e0.elapsed_time(e1) / reps
        vendor = {"what": "torch.nn.functional.scaled_dot_product_attention, flash / memory-efficient "
                          "backends only, [B][H][S][D] contiguous bf16, forward + backward, same run",
                  "ms": round(vms, 3), "tflops": round((ff + fb) / (vms * 1e-3) / 1e12, 1),
                  "achieved_over_vendor": round(vms / ms, 4)}
        del qt, kt, vt, dyt
    except Exception as e:  # backend unavailable on this build: report why
        vendor = {"what": "torch SDPA fused backends", "error": f"{type(e).__name__}: {e}"[:200]}
    del q, k, v, dy
    torch.cuda.empty_cache()
    return {"metric": "attention TFLOP/s (forward + backward, algorithmic flops)",
            "value": round(tflops, 1), "unit": "TFLOP/s", "dtype": "bf16",
            "config": {"workload": "wan2.1-14b self-attention of one block: B=1, 32760 tokens, "
                                   "40 heads x 128, no mask, not causal", "flops_fwd": ff,
                       "flops_bwd": fb},
            "ms": round(ms, 3), "fwd_ms": round(fwd_ms, 3), "bwd_ms": round(bwd_ms, 3),
            "kernels": {n: {"launches": c // reps, "avg_ms": round(t / c, 4)} for n, (c, t) in kern.items()},
            "roofline": {"kernel": "attn_fwd_kernel, attn_dkdv32_kernel (attn_dkdv_kernel for few keys), attn_dq_kernel", "bound": "mfma",
                         "achieved": round(tflops, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                         "fwd": round(ff / (fwd_ms * 1e-3) / 1e12, 1),
                         "bwd": round(fb / (bwd_ms * 1e-3) / 1e12, 1)},
            "vendor_sdpa": vendor}


def attention_cpu_baseline(seconds=5.0):
    """The reference's CPU attention (memory_efficient_attention with its backward,
    attention.jl:106-221: f32 128 x 128 score tiles on BLAS, online softmax) restated in
    oracle/cpu_path.py on torch's CPU BLAS with every thread this process has, timed on a bounded
    sample: one head of the Wan-14B shape, all 32760 keys, as many queries as fit the time."""
    import torch
    from oracle import cpu_path
    B, S, H, D = ATT_SHAPE
    threads = torch.get_num_threads()
    g = torch.Generator().manual_seed(3)
    k = torch.randn((S, D), generator=g)
    v = torch.randn((S, D), generator=g)
    nq = 128
    while True:
        q = torch.randn((nq, D), generator=g)
        dy = torch.randn((nq, D), generator=g)
        t0 = time.perf_counter()
        out, lse = cpu_path.attention_forward(q, k, v)
        cpu_path.attention_backward(q, k, v, dy, out, lse)
        dt = time.perf_counter() - t0
        if dt > seconds / 3 or nq >= 8192:
            break
        nq *= 2
    ff, fb = attention_flops(1, nq, S, 1, D)
    return {"value": round((ff + fb) / dt / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "host": host_info(),
            "sample": f"one head, {nq} queries x {S} keys x {D}, forward + backward, the reference's "
                      f"f32 128x128-tiled algorithm on torch CPU BLAS ({threads} threads), {dt:.2f} s"}


def copy_gbs(dev, nbytes=4 << 30, reps=5):
    """Device-to-device copy bandwidth (bytes read + written per second): the practical ceiling
    of a streaming kernel that reads and writes HBM, measured in the same run."""
    import torch
    a = torch.empty((nbytes,), dtype=torch.uint8, device=dev).fill_(3)
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del a, b
    torch.cuda.empty_cache()
    return 2.0 * nbytes / (ms * 1e-3) / 1e9


def host_info():
    """The host CPU the baselines run on: model, logical CPUs, CPUs this process may use."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def device_info(dev, sclk=None):
    """The GPU: name, compute units, architecture, and (when the driver's sysfs file is readable)
    the shader clock level it sat at when sampled (right after the timed steps)."""
    import torch
    p = torch.cuda.get_device_properties(dev)
    return {"name": torch.cuda.get_device_name(dev), "compute_units": p.multi_processor_count, "arch": p.gcnArchName,
            "sclk_after_timed_steps": sclk}


def read_sclk(dev):
    """The current shader clock level from /sys/bus/pci/devices/<this GPU>/pp_dpm_sclk (the line
    marked '*'), or None where the file is missing or unreadable."""
    import torch
    try:
        p = torch.cuda.get_device_properties(dev)
        path = f"/sys/bus/pci/devices/{p.pci_domain_id:04x}:{p.pci_bus_id:02x}:{p.pci_device_id:02x}.0/pp_dpm_sclk"
        with open(path) as f:
            cur = [l.split(":", 1)[1].replace("*", "").strip() for l in f if "*" in l]
        return cur[0] if cur else None
    except (OSError, IndexError, AttributeError, RuntimeError):
        return None


def pack_cpu_baseline(samples, seconds=5.0):
    """The reference packs on the host CPU (quantize_frozen_matrix, quantization.jl:35-44 on
    Float32.(Array(W))); the oracle's C restatement (OpenMP) is timed on a sample of 14B rows.
    The same leg compares the sampled rows of every timed GPU launch with the oracle bit for bit."""
    import numpy as np
    import oracle
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    checked = 0
    for (wb, qg, sg, rows, K) in samples:
        qo, so, st = oracle.pack(wb.view(np.uint16), "bf16")
        if st != 0 or not np.array_equal(qo, qg) or not np.array_equal(so.view(np.uint32),
                                                                         sg.view(np.uint32)):
            raise SystemExit(f"pack: sampled rows of the {rows}x{K} launch differ from the oracle")
        checked += len(qg)
    rows = 2048
    w = oracle.normal_bf16(5, (rows, 5120), 0.02, outlier_rate=1e-3)
    t0 = time.perf_counter(); oracle.pack(w, "bf16"); t1 = time.perf_counter()
    reps = max(1, int(seconds / max(t1 - t0, 1e-6)))
    t0 = time.perf_counter()
    for _ in range(reps):
        oracle.pack(w, "bf16")
    t1 = time.perf_counter()
    nbytes = 3 * rows * 5120 + 4 * rows
    return {"value": round(nbytes * reps / (t1 - t0) / 1e9, 2), "unit": "GB/s", "cores": threads,
            "kind": "port", "host": host_info(),
            "sample": f"{rows}x5120 bf16 rows x {reps} repetitions, C oracle "
                      f"(OpenMP, {threads} threads), {t1 - t0:.2f} s",
            "gpu_rows_checked_bit_exact": checked}


class Projection:
    def __init__(self, name, K, N, M, r, dev, gen, act=None, alpha=ALPHA):
        import torch
        from reels_amd import quantize_frozen_matrix, workspace_bytes, _lib
        self.name, self.K, self.N, self.M, self.r = name, K, N, M, r
        bf = act or torch.bfloat16
        w = torch.randn((N, K), generator=gen, device=dev, dtype=torch.float32).mul_(0.02)
        self.W = quantize_frozen_matrix(w.to(bf), bf)
        del w
        self.x = torch.randn((M, K), generator=gen, device=dev, dtype=torch.float32).to(bf)
        self.dy = torch.randn((M, N), generator=gen, device=dev, dtype=torch.float32).to(bf)
        self.A = (torch.randn((K, r), generator=gen, device=dev) * 0.01).to(bf)
        self.B = (torch.randn((r, N), generator=gen, device=dev) * 0.01).to(bf)
        self.y = torch.empty((M, N), dtype=bf, device=dev)
        self.h = torch.empty((M, r), dtype=bf, device=dev)
        self.dx = torch.empty((M, K), dtype=bf, device=dev)
        self.dA = torch.empty((K, r), dtype=torch.float32, device=dev)
        self.dB = torch.empty((r, N), dtype=torch.float32, device=dev)
        self.wsf_n = workspace_bytes(M, K, N, r, _lib.WS_FWD, bf)
        self.wsb_n = workspace_bytes(M, K, N, r, _lib.WS_BWD, bf)
        self.wsf = torch.empty((self.wsf_n,), dtype=torch.uint8, device=dev)
        self.wsb = torch.empty((self.wsb_n,), dtype=torch.uint8, device=dev)
        c = float(torch.tensor(alpha, dtype=torch.float32) / torch.tensor(float(r)))
        p = lambda t: ctypes.c_void_p(t.data_ptr())
        st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        self.fwd_args = (p(self.x), p(self.W.values), p(self.W.scales), p(self.A), p(self.B), None,
                         M, K, N, r, c, p(self.y), p(self.h), p(self.wsf), self.wsf_n, st)
        self.bwd_args = (p(self.dy), p(self.x), p(self.h), p(self.W.values), p(self.W.scales),
                         p(self.A), p(self.B), M, K, N, r, c, p(self.dx), p(self.dA), p(self.dB),
                         p(self.wsb), self.wsb_n, st)


def run_step(L, projs, check, sfx="", streamer=None):
    fwd, bwd = getattr(L, "reels_hip_i8lora_fwd" + sfx), getattr(L, "reels_hip_i8lora_bwd" + sfx)
    if streamer is None:
        for pr in projs:
            check("reels_hip_i8lora_fwd" + sfx, fwd(*pr.fwd_args))
        for pr in reversed(projs):
            check("reels_hip_i8lora_bwd" + sfx, bwd(*pr.bwd_args))
        return
    # offloaded weights: each projection's codes arrive in a device slot while the previous
    # projection computes; the call takes the slot's pointers
    from reels_amd.offload import run_streamed
    p = lambda t: ctypes.c_void_p(t.data_ptr())

    def f(i, W):
        a = list(projs[i].fwd_args); a[1], a[2] = p(W.values), p(W.scales)
        check("reels_hip_i8lora_fwd" + sfx, fwd(*a))

    rev = list(reversed(projs))

    def b(i, W):
        a = list(rev[i].bwd_args); a[3], a[4] = p(W.values), p(W.scales)
        check("reels_hip_i8lora_bwd" + sfx, bwd(*a))

    run_streamed([pr.Wh for pr in projs], f, streamer)
    run_streamed([pr.Wh for pr in rev], b, streamer)


PROJECTIONS_13B = [("self_attn.q", 1536, 1536), ("self_attn.k", 1536, 1536),
                   ("self_attn.v", 1536, 1536), ("self_attn.o", 1536, 1536),
                   ("ffn.0", 1536, 8960), ("ffn.2", 8960, 1536)]


def _time_ms(fn, reps, warmup=2, warm_s=0.0):
    """Mean ms of fn over reps calls between two events on torch's current stream (the stream the
    library launches on), after warmup untimed calls and then, for calls of tens of microseconds,
    untimed calls for at least warm_s seconds: the GPU's clocks ramp up over the first ~10 ms of
    back-to-back work after an idle spell (a 512-token forward on 5120 x 5120 ran 41.5 us in its
    first 50 launches and 34.2 us from the 300th on), so short calls are timed at steady clocks,
    ours and the vendor's alike."""
    import time
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < warm_s:
        for _ in range(50):
            fn()
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


class Chain:
    """Config 4: a stack of Wan-2.1-1.3B layers, each q -> k -> v -> o -> ffn.0 -> gelu_tanh ->
    ffn.2 (dim 1536, ffn 8960; src/models/wan21/transformer.jl:289-292), LoRA r = 32 (alpha 32)
    on every linear. One step = the forward through every layer (each linear's input kept, as
    the backward needs it) and the backward in reverse: dX chained back through the GELU
    pullback, dA and dB for every linear. Every buffer is allocated up front."""

    def __init__(self, dev, gen, layers=30, M=TOKENS, r=RANK, D=1536, F=8960):
        import torch
        from reels_amd import _lib, quantize_frozen_matrix, workspace_bytes
        bf = torch.bfloat16
        self.M, self.r, self.layers = M, r, layers
        p = lambda t: ctypes.c_void_p(t.data_ptr())
        self.st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        shapes = [(D, D)] * 4 + [(D, F), (F, D)]
        c = float(torch.tensor(ALPHA, dtype=torch.float32) / torch.tensor(float(r)))
        wsf = max(workspace_bytes(M, K, N, r, _lib.WS_FWD) for (K, N) in shapes)
        wsb = max(workspace_bytes(M, K, N, r, _lib.WS_BWD) for (K, N) in shapes)
        self.wsf = torch.empty((wsf,), dtype=torch.uint8, device=dev)
        self.wsb = torch.empty((wsb,), dtype=torch.uint8, device=dev)
        self.x0 = torch.randn((M, D), generator=gen, device=dev).to(bf)
        self.gout = torch.randn((M, D), generator=gen, device=dev).to(bf)
        # two gradient buffers per width, used alternately down the chain
        pool = {D: [torch.empty((M, D), dtype=bf, device=dev) for _ in range(2)],
                F: [torch.empty((M, F), dtype=bf, device=dev) for _ in range(2)]}
        self.keep = [pool]
        self.links = []
        cur = self.x0
        for li in range(layers):
            for j, (K, N) in enumerate(shapes):
                w = (torch.randn((N, K), generator=gen, device=dev) * 0.02).to(bf)
                W = quantize_frozen_matrix(w, bf)
                del w
                A = (torch.randn((K, r), generator=gen, device=dev) * 0.01).to(bf)
                B = (torch.randn((r, N), generator=gen, device=dev) * 0.01).to(bf)
                y = torch.empty((M, N), dtype=bf, device=dev)
                h = torch.empty((M, r), dtype=bf, device=dev)
                gl = torch.empty((M, N), dtype=bf, device=dev) if j == 4 else None
                dA = torch.empty((K, r), dtype=torch.float32, device=dev)
                dB = torch.empty((r, N), dtype=torch.float32, device=dev)
                self.keep.append((W, A, B, y, h, gl, dA, dB))
                gx = self.links[-1]["y"] if j == 5 else None  # ffn.2's input is gelu(ffn.0's y)
                self.links.append(dict(
                    K=K, N=N, gelu=j == 4, after_gelu=j == 5, x=cur, y=y, gl=gl,
                    fwd=(p(cur), p(W.values), p(W.scales), p(A), p(B), None, M, K, N, r, c, p(y),
                         p(h), p(self.wsf), wsf, self.st),
                    fwd_gelu=(p(cur), p(W.values), p(W.scales), p(A), p(B), None, M, K, N, r, c,
                              p(y), p(gl), p(h), p(self.wsf), wsf, self.st) if j == 4 else None,
                    bwd=lambda dy, dx, x=cur, W=W, A=A, B=B, h=h, dA=dA, dB=dB, K=K, N=N: (
                        p(dy), p(x), p(h), p(W.values), p(W.scales), p(A), p(B), M, K, N, r, c,
                        p(dx), p(dA), p(dB), p(self.wsb), wsb, self.st),
                    bwd_gelu=lambda dy, dx, x=cur, W=W, A=A, B=B, h=h, dA=dA, dB=dB, K=K, N=N, gx=gx: (
                        p(dy), p(x), p(h), p(W.values), p(W.scales), p(A), p(B), p(gx), M, K, N,
                        r, c, p(dx), p(dA), p(dB), None, p(self.wsb), wsb, self.st)))
                cur = gl if j == 4 else y
        # the backward's buffer sequence, fixed once: dy of each link and its dx buffer; with the
        # GELU's pullback as a separate call (plan_sep) or fused into ffn.2's dX (plan)
        self.plan_sep, self.plan = [], []
        gd = self.gout
        for lk in reversed(self.links):
            pre = None
            if lk["gelu"]:  # the pullback of gelu_tanh before ffn.0's backward
                g2 = next(t for t in pool[lk["N"]] if t is not gd)
                pre = (p(lk["y"]), p(gd), p(g2), M * lk["N"])
                gd = g2
            dx = next(t for t in pool[lk["K"]] if t is not gd)
            self.plan_sep.append((lk, pre, lk["bwd"](gd, dx)))
            gd = dx
        gd = self.gout
        for lk in reversed(self.links):
            dx = next(t for t in pool[lk["K"]] if t is not gd)
            self.plan.append((lk, lk["bwd_gelu"](gd, dx) if lk["after_gelu"] else lk["bwd"](gd, dx)))
            gd = dx
        self.flops = layers * sum(linear_flops(M, K, N, r) for (K, N) in shapes)

    def step(self, L, check, fused=True):
        for lk in self.links:
            if lk["gelu"] and fused:
                check("reels_hip_i8lora_fwd_gelu", L.reels_hip_i8lora_fwd_gelu(*lk["fwd_gelu"]))
                continue
            check("reels_hip_i8lora_fwd", L.reels_hip_i8lora_fwd(*lk["fwd"]))
            if lk["gelu"]:
                check("reels_hip_gelu_tanh", L.reels_hip_gelu_tanh(
                    ctypes.c_void_p(lk["y"].data_ptr()), ctypes.c_void_p(lk["gl"].data_ptr()),
                    self.M * lk["N"], self.st))
        if fused:
            for (lk, args) in self.plan:
                if lk["after_gelu"]:
                    check("reels_hip_i8lora_bwd_gelu", L.reels_hip_i8lora_bwd_gelu(*args))
                else:
                    check("reels_hip_i8lora_bwd", L.reels_hip_i8lora_bwd(*args))
            return
        for (lk, pre, args) in self.plan_sep:
            if pre is not None:
                check("reels_hip_gelu_tanh_bwd", L.reels_hip_gelu_tanh_bwd(*pre, self.st))
            check("reels_hip_i8lora_bwd", L.reels_hip_i8lora_bwd(*args))


def configs_bench(dev, L, check, which=("cfg1", "cfg2", "cfg4", "cfg5a")):
    """The smaller int8 LoRA workloads on this GPU, each as TFLOP/s of forward + dX + dA + dB
    (4MNK + 6Mr(K+N) per linear): config 1 (one 1536 x 1536 linear, 1024 tokens, r 16, alpha 16),
    config 2 (the six Wan-2.1-1.3B block projections at 32760 tokens), config 4 (the 30-layer
    1.3B chain with GELU), and config 5a (cross-attention K/V 5120 -> 5120 at 77 / 333 / 512 text
    tokens, forward and backward timed separately, as HBM GB/s of their algorithmic bytes)."""
    import torch
    out = {}
    gen = torch.Generator(device=dev).manual_seed(99)
    if "cfg1" in which:
        out.update(_cfg1(dev, L, check, gen))
    if "cfg2" in which:
        out.update(_cfg2(dev, L, check, gen))
    if "cfg4" in which:
        out.update(_cfg4(dev, L, check, gen))
    if "cfg5a" in which:
        out.update(_cfg5a(dev, L, check, gen))
    torch.cuda.empty_cache()
    return out


def _cfg1(dev, L, check, gen):
    out = {}
    pr = Projection("cfg1", 1536, 1536, 1024, 16, dev, gen, alpha=16.0)
    ms = _time_ms(lambda: run_step(L, [pr], check), reps=300, warmup=5, warm_s=WARM_S)
    f = linear_flops(1024, 1536, 1536, 16)
    out["cfg1"] = {"what": "one int8 LoRA linear 1536 -> 1536, 1024 tokens, r 16, alpha 16, "
                           "fwd + dX + dA + dB", "ms": round(ms, 4),
                   "tflops": round(f / (ms * 1e-3) / 1e12, 1)}
    return out


def _cfg2(dev, L, check, gen):
    import torch
    out = {}
    projs = [Projection(n, K, N, TOKENS, RANK, dev, gen) for (n, K, N) in PROJECTIONS_13B]
    ms = _time_ms(lambda: run_step(L, projs, check), reps=10)
    f = sum(linear_flops(TOKENS, K, N, RANK) for (_, K, N) in PROJECTIONS_13B)
    out["cfg2"] = {"what": "wan2.1-1.3b block projections q/k/v/o 1536 -> 1536, ffn 1536 -> 8960 "
                           "-> 1536 at 32760 tokens, r 32, fwd + dX + dA + dB", "ms": round(ms, 3),
                   "tflops": round(f / (ms * 1e-3) / 1e12, 1),
                   "frac_of_bf16_peak": round(f / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                   "gemm_vs_vendor": _cfg2_gemms(dev, L, check, projs)}
    del projs
    torch.cuda.empty_cache()
    return out


def _cfg2_gemms(dev, L, check, projs, reps=20):
    """Per config-2 shape: the library's GEMM launches alone (HIP events around each launch,
    forward and dX) against torch.matmul's bf16 GEMM (the vendor library) on the same operand
    shapes and layouts: x [M][K] by a [N][K] weight transposed (forward), dy [M][N] by the
    [N][K] weight (dX). us per launch; ratio = vendor time / ours (above 1: ours faster)."""
    import torch
    from reels_amd import _lib
    res = {}
    for name in ("self_attn.q", "ffn.0", "ffn.2"):
        pr = next(p for p in projs if p.name == name)
        t = {}
        for mode, fn, args in (("fwd", L.reels_hip_i8lora_fwd, pr.fwd_args),
                               ("dx", L.reels_hip_i8lora_bwd, pr.bwd_args)):
            call = lambda: check("reels_hip_i8lora_" + ("fwd" if mode == "fwd" else "bwd"), fn(*args))
            call()
            torch.cuda.synchronize()
            _lib.check("reels_hip_trace_only", L.reels_hip_trace_only(b"gemm_kernel"))
            _lib.check("reels_hip_trace_start", L.reels_hip_trace_start(8 * reps))
            for _ in range(reps):
                call()
            torch.cuda.synchronize()
            recs = [ms for (n, ms) in _lib.trace_records() if n.endswith("<0>" if mode == "fwd" else "<1>")]
            t[mode] = sum(recs) / max(len(recs), 1) * 1e3
        _lib.check("reels_hip_trace_only", L.reels_hip_trace_only(b""))
        w = torch.randn((pr.N, pr.K), device=dev).to(torch.bfloat16)
        vf = _time_ms(lambda: torch.matmul(pr.x, w.t()), reps=reps) * 1e3
        vd = _time_ms(lambda: torch.matmul(pr.dy, w), reps=reps) * 1e3
        del w
        fl = 2.0 * pr.M * pr.K * pr.N
        res[f"{pr.K}x{pr.N}"] = {
            "fwd_us": round(t["fwd"], 1), "vendor_fwd_us": round(vf, 1),
            "fwd_ratio": round(vf / t["fwd"], 3), "dx_us": round(t["dx"], 1),
            "vendor_dx_us": round(vd, 1), "dx_ratio": round(vd / t["dx"], 3),
            "fwd_tflops": round(fl / (t["fwd"] * 1e-6) / 1e12, 1),
            "vendor_fwd_tflops": round(fl / (vf * 1e-6) / 1e12, 1)}
    return res


def _cfg4(dev, L, check, gen):
    import torch
    out = {}
    ch = Chain(dev, gen)
    ms = _time_ms(lambda: ch.step(L, check), reps=3, warmup=1)
    ms_sep = _time_ms(lambda: ch.step(L, check, fused=False), reps=3, warmup=1)
    out["cfg4"] = {"what": "30 wan2.1-1.3b layers (q -> k -> v -> o -> ffn.0 -> gelu_tanh -> "
                           "ffn.2) at 32760 tokens, r 32: one forward then one backward through "
                           "the chain (dX chained, dA and dB per linear); the GELU fused into "
                           "ffn.0's forward epilogue (reels_hip_i8lora_fwd_gelu) and its pullback "
                           "into ffn.2's dX (reels_hip_i8lora_bwd_gelu)", "ms": round(ms, 2),
                   "ms_separate_gelu_passes": round(ms_sep, 2),
                   "tflops": round(ch.flops / (ms * 1e-3) / 1e12, 1),
                   "frac_of_bf16_peak": round(ch.flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                   "flops": ch.flops}
    del ch
    torch.cuda.empty_cache()
    return out


def _cfg5a(dev, L, check, gen):
    out = {}
    sk = {}
    for M in (77, 333, 512):
        K = N = 5120
        pr = Projection("cross_kv", K, N, M, RANK, dev, gen)
        fms = _time_ms(lambda: check("reels_hip_i8lora_fwd", L.reels_hip_i8lora_fwd(*pr.fwd_args)),
                       reps=300, warmup=5, warm_s=WARM_S)
        bms = _time_ms(lambda: check("reels_hip_i8lora_bwd", L.reels_hip_i8lora_bwd(*pr.bwd_args)),
                       reps=300, warmup=5, warm_s=WARM_S)
        fb = 2 * M * K + N * K + 4 * N + 2 * M * N + 2 * M * RANK
        bb = 2 * M * N + N * K + 4 * N + 4 * M * K + 2 * M * RANK
        ff = 2.0 * M * N * K + 2.0 * M * RANK * (K + N)
        bf_ = 2.0 * M * N * K + 4.0 * M * RANK * (K + N)
        # the vendor library's plain bf16 GEMM on the same shape (bf16 weight, no scales, no LoRA)
        import torch
        xv = torch.randn((M, K), device=dev, dtype=torch.bfloat16)
        wv = torch.randn((N, K), device=dev, dtype=torch.bfloat16)
        vms = _time_ms(lambda: torch.matmul(xv, wv.t()), reps=300, warmup=5, warm_s=WARM_S)
        del xv, wv
        sk[str(M)] = {"fwd_us": round(fms * 1e3, 2), "bwd_us": round(bms * 1e3, 2),
                      "vendor_bf16_gemm_us": round(vms * 1e3, 2),
                      "fwd_gbs": round(fb / (fms * 1e-3) / 1e9, 1),
                      "bwd_gbs": round(bb / (bms * 1e-3) / 1e9, 1),
                      "fwd_frac_of_hbm": round(fb / (fms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                      "fwd_tflops": round(ff / (fms * 1e-3) / 1e12, 1),
                      "bwd_tflops": round(bf_ / (bms * 1e-3) / 1e12, 1),
                      "fwd_bytes": fb, "bwd_bytes": bb}
        sk[str(M)].update(_cfg5a_rotating(dev, L, check, gen, M, K, N, fb))
        del pr
    out["cfg5a"] = {"what": "cross-attention K/V projection 5120 -> 5120, r 32, at 77 / 333 / 512 "
                            "text tokens; bytes = 2MK + NK + 4N + 2MN + 2Mr (fwd), 2MN + NK + 4N "
                            "+ 4MK + 2Mr (bwd); peak 8 TB/s; vendor_bf16_gemm_us: torch.matmul of "
                            "the same x by a bf16 weight (twice the weight bytes, no scales or LoRA)",
                    "tokens": sk}
    return out


def _cfg5a_rotating(dev, L, check, gen, M, K, N, fb, nw=12, reps=48):
    """The forward over a rotating set of nw weights (12 x 26 MB int8 = 315 MB, above the 256 MB
    last-level cache, so each call reads its weight from HBM), against torch.matmul over 12 bf16
    weights (629 MB) of the same shape."""
    import torch
    prs = [Projection("cross_kv", K, N, M, RANK, dev, gen) for _ in range(nw)]
    i = [0]

    def ours():
        check("reels_hip_i8lora_fwd", L.reels_hip_i8lora_fwd(*prs[i[0] % nw].fwd_args))
        i[0] += 1
    fms = _time_ms(ours, reps=reps, warmup=nw, warm_s=WARM_S)
    x = prs[0].x
    ws = [torch.randn((N, K), device=dev).to(torch.bfloat16) for _ in range(nw)]

    def vend():
        torch.matmul(x, ws[i[0] % nw].t())
        i[0] += 1
    vms = _time_ms(vend, reps=reps, warmup=nw, warm_s=WARM_S)
    del prs, ws
    torch.cuda.empty_cache()
    return {"rotating_fwd_us": round(fms * 1e3, 2), "rotating_vendor_us": round(vms * 1e3, 2),
            "rotating_fwd_gbs": round(fb / (fms * 1e-3) / 1e9, 1),
            "rotating_note": f"{nw} weights in turn (int8 {nw * N * K / 1e6:.0f} MB, vendor bf16 "
                             f"{2 * nw * N * K / 1e6:.0f} MB): weight reads from HBM"}


def configs_cpu_baseline(configs):
    """The reference's CPU path (oracle/cpu_path.py: fp32 materialised dequant + torch CPU BLAS)
    on the smaller configurations, beside their GPU figures: config 1 in full, one linear of each
    config-2 shape at 32760 tokens, config 5a in full (forward and backward timed apart)."""
    import torch
    from oracle import cpu_path
    threads = torch.get_num_threads()
    out = {"kind": "port", "cores": threads, "host": host_info(),
           "what": "fp32 materialised dequant + torch CPU BLAS, all host threads; configs 1 and "
                   "5a: best of three runs after an untimed one, config 2: one run per shape"}
    if "cfg1" in configs:
        tf, tb = cpu_path.time_linear(1536, 1536, 1024, 16, reps=3)
        ms = (tf + tb) * 1e3
        f = linear_flops(1024, 1536, 1536, 16)
        out["cfg1"] = {"ms": round(ms, 3), "tflops": round(f / (ms * 1e-3) / 1e12, 4),
                       "gpu_speedup": round(ms / configs["cfg1"]["ms"], 1)}
    if "cfg2" in configs:
        shapes = {}
        for (name, K, N) in (("q", 1536, 1536), ("ffn.0", 1536, 8960), ("ffn.2", 8960, 1536)):
            tf, tb = cpu_path.time_linear(K, N, TOKENS, RANK, warm=0)  # one timed run
            f = linear_flops(TOKENS, K, N, RANK)
            shapes[name] = {"ms": round((tf + tb) * 1e3, 1),
                            "tflops": round(f / (tf + tb) / 1e12, 4)}
        out["cfg2_one_linear_per_shape"] = shapes
    if "cfg5a" in configs:
        tok = {}
        for M in (77, 333, 512):
            tf, tb = cpu_path.time_linear(5120, 5120, M, RANK, reps=3)
            g = configs["cfg5a"]["tokens"][str(M)]
            tok[str(M)] = {"fwd_us": round(tf * 1e6, 1), "bwd_us": round(tb * 1e6, 1),
                           "gpu_speedup_fwd": round(tf * 1e6 / g["fwd_us"], 1),
                           "gpu_speedup_bwd": round(tb * 1e6 / g["bwd_us"], 1)}
        out["cfg5a"] = tok
    return out


def cpu_baseline(seconds):
    """The reference's CPU path (fp32: dequantize-materialise + BLAS sgemm + rank-r GEMMs, see
    oracle/cpu_path.py) on a bounded sample of the same six projections at fewer tokens."""
    import torch
    from oracle import cpu_path
    threads = torch.get_num_threads()
    shapes = [(K, N) for (_, K, N) in PROJECTIONS]
    t_cal, f_cal = cpu_path.time_block(shapes, 128, RANK)
    rate = f_cal / max(t_cal, 1e-9)
    per_token = f_cal / 128
    m = int(seconds * rate / per_token) // 128 * 128
    m = max(128, min(m, TOKENS))
    t, f = cpu_path.time_block(shapes, m, RANK, seed=1)
    return {"value": round(f / t / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "host": host_info(),
            "sample": (f"Wan-14B block projections (q,k,v,o 5120->5120, ffn 5120->13824->5120), "
                       f"r=32, fwd+dX+dA+dB at {m} tokens (of {TOKENS}), fp32 materialised "
                       f"dequant + torch CPU BLAS, {threads} threads, {t:.2f} s")}


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on exactly one GPU (asked for --gpus {args.gpus}, WORLD_SIZE "
              f"{world}); the multi-GPU path is not built", file=sys.stderr)
        sys.exit(2)
    import torch
    from reels_amd import _lib
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate_copy:
        a = torch.empty((1 << 30,), dtype=torch.uint8, device=dev).fill_(1)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print("copied 3 x 1 GiB device to device")
        return
    L = _lib.lib()
    if args.pack_only:
        print(json.dumps({"pack": pack_bench(dev)[0]}))
        return
    if args.configs_only:
        which = tuple(args.configs_only.split(","))
        print(json.dumps({"configs": configs_bench(dev, L, _lib.check, which)}))
        return
    if args.attention_only:
        att = attention_bench(dev)
        if args.cpu_seconds > 0:
            att["cpu_baseline"] = attention_cpu_baseline(min(5.0, args.cpu_seconds))
        print(json.dumps({"attention": att}))
        return
    gen = torch.Generator(device=dev).manual_seed(1234)
    M = args.tokens
    act = {"f16": torch.float16, "f32": torch.float32}.get(args.dtype, torch.bfloat16)
    sfx = {"f16": "_f16", "f32": "_f32"}.get(args.dtype, "")
    projs = [Projection(n, K, N, M, RANK, dev, gen, act) for (n, K, N) in PROJECTIONS]
    streamer = None
    if args.offload != "none":
        from reels_amd.offload import PerCallUploader, WeightStreamer, offload_weight
        for pr in projs:
            pr.Wh = offload_weight(pr.W)
            pr.W = None
        torch.cuda.empty_cache()
        streamer = WeightStreamer(dev, slots=2) if args.offload == "stream" else PerCallUploader(dev)
    torch.cuda.synchronize()

    for _ in range(args.warmup):
        run_step(L, projs, _lib.check, sfx, streamer)
    torch.cuda.synchronize()

    # count one step's launches (an untimed traced step) to size the trace buffer exactly
    _lib.check("reels_hip_trace_only", L.reels_hip_trace_only(b"gemm_kernel" if args.trace == "gemm" else b""))
    _lib.check("reels_hip_trace_start", L.reels_hip_trace_start(4096))
    run_step(L, projs, _lib.check, sfx, streamer)
    torch.cuda.synchronize()
    launches_per_step = len(_lib.trace_records())
    _lib.check("reels_hip_trace_start", L.reels_hip_trace_start(launches_per_step * args.steps))
    torch.cuda.synchronize()
    up0 = streamer.uploads if streamer else 0
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run_step(L, projs, _lib.check, sfx, streamer)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    sclk = read_sclk(dev)
    recs = _lib.trace_records()
    all_recs, all_steps = recs, args.steps
    if args.trace == "gemm":
        # the per-kernel breakdown: one more (untimed) step with every kernel traced
        _lib.check("reels_hip_trace_only", L.reels_hip_trace_only(b""))
        _lib.check("reels_hip_trace_start", L.reels_hip_trace_start(4096))
        run_step(L, projs, _lib.check, sfx, streamer)
        torch.cuda.synchronize()
        all_recs, all_steps = _lib.trace_records(), 1
    offload = None
    if streamer is not None:
        ups = (streamer.uploads - up0) / args.steps
        per = {id(pr.Wh): pr.Wh.values.numel() + 4 * pr.Wh.scales.numel() for pr in projs}
        nbytes = sum(per.values()) * ups / len(projs)  # mean bytes per upload x uploads
        step_s = (t1 - t0) / args.steps
        offload = {"what": ("int8 codes + f32 scales in pinned host memory, uploaded one "
                            "projection ahead on a copy stream (WeightStreamer, 2 slots)")
                           if args.offload == "stream" else
                           ("int8 codes + f32 scales in pinned host memory, copied on the compute "
                            "stream right before each use (per-call upload, no overlap)"),
                   "uploads_per_step": ups, "h2d_bytes_per_step": int(nbytes),
                   "h2d_gbs_over_step": round(nbytes / step_s / 1e9, 2)}

    ms_per_step = (t1 - t0) * 1e3 / args.steps
    step_flops = sum(linear_flops(M, K, N, RANK) for (_, K, N) in PROJECTIONS)
    value = step_flops / (ms_per_step * 1e-3) / 1e12

    # per-kernel statistics from the event trace (launch order is fixed within a step)
    per_step = len(recs) // max(args.steps, 1)
    kern = {}
    for name, ms in all_recs:
        d = kern.setdefault(name, [0, 0.0])
        d[0] += 1
        d[1] += ms
    gemm_ms = {"fwd": 0.0, "dx": 0.0}
    gemm_n = {"fwd": 0, "dx": 0}
    gemm_fl = {"fwd": 0.0, "dx": 0.0}
    for step in range(args.steps):
        rs = recs[step * per_step:(step + 1) * per_step]
        fi = [ms for (n, ms) in rs if "gemm_kernel" in n and n.endswith("<0>")]
        bi = [ms for (n, ms) in rs if "gemm_kernel" in n and n.endswith("<1>")]
        for (pr, ms) in zip(projs, fi):
            gemm_ms["fwd"] += ms; gemm_n["fwd"] += 1
            gemm_fl["fwd"] += gemm_flops("fwd", M, pr.K, pr.N, RANK)
        for (pr, ms) in zip(reversed(projs), bi):
            gemm_ms["dx"] += ms; gemm_n["dx"] += 1
            gemm_fl["dx"] += gemm_flops("dx", M, pr.K, pr.N, RANK)
    tot_ms = gemm_ms["fwd"] + gemm_ms["dx"]
    achieved = (gemm_fl["fwd"] + gemm_fl["dx"]) / (tot_ms * 1e-3) / 1e12 if tot_ms > 0 else 0.0
    gemm_names = sorted({n for (n, _) in recs if "gemm_kernel" in n})
    vendor = vendor_gemm_tflops(dev, M, 5120, 5120, dtype=act)
    deq = {"bf16": "bf16(q*s)", "f16": "f16(q*f16(s))", "f32": "fl32(q*s)"}[args.dtype]
    peak = PEAK_TFLOPS[args.dtype]
    roofline = {
        "kernel": " + ".join(gemm_names) + f" (<0> fwd, <1> dX; {args.dtype} MFMA on the "
                                           f"dequantized weight {deq})",
        "bound": "mfma", "achieved": round(achieved, 2), "peak": peak,
        "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
        "traffic": GEMM_TRAFFIC_BYTES,
        "traffic_note": GEMM_TRAFFIC_NOTE,
        "avg_launch_ms": {k: round(gemm_ms[k] / max(gemm_n[k], 1), 4) for k in gemm_ms},
        "launches": gemm_n,
        "vendor_bf16_gemm": {"what": f"torch.matmul {args.dtype} (vendor library), {M}x5120 by 5120x5120, "
                                     "sustained ~1.5 s loop, same run", "tflops": round(vendor, 1),
                             "achieved_over_vendor": round(achieved / vendor, 4)},
    }
    kernels = {n: {"launches_per_step": c // all_steps, "avg_ms": round(t / c, 4),
                   "ms_per_step": round(t / all_steps, 4)}
               for n, (c, t) in sorted(kern.items(), key=lambda kv: -kv[1][1])}

    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline(args.cpu_seconds)
    del projs
    torch.cuda.empty_cache()
    configs = None
    if not args.no_configs and args.dtype == "bf16" and args.offload == "none":
        configs = configs_bench(dev, L, _lib.check)
        if args.cpu_seconds > 0:
            configs["cpu_baseline"] = configs_cpu_baseline(configs)
    pack = None
    if not args.no_pack:
        pack, samples = pack_bench(dev)
        if args.cpu_seconds > 0:
            pack["cpu_baseline"] = pack_cpu_baseline(samples, min(5.0, args.cpu_seconds))
    att = None
    if not args.no_attention and args.dtype == "bf16" and args.offload == "none":
        att = attention_bench(dev)
        if args.cpu_seconds > 0:
            att["cpu_baseline"] = attention_cpu_baseline(min(5.0, args.cpu_seconds))

    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": args.dtype,
        "data": "synthetic",
        "config": {"workload": "wan2.1-14b block projections: self_attn q/k/v/o 5120->5120, "
                               "ffn 5120->13824->5120; int8 per-channel frozen weights; LoRA "
                               "r=32 alpha=32; forward + dX + dA + dB",
                   "tokens": M, "rank": RANK, "flops_per_step": step_flops,
                   "weights": {"none": "resident in HBM", "stream": "cpu_offload (pinned host, "
                               "streamed)", "sync": "cpu_offload (pinned host, per-call upload)"}
                              [args.offload]},
        "offload": offload,
        "frac_of_bf16_peak": round(value / PEAK_BF16_TFLOPS, 4),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kernels,
        "kernels_from": ("one extra untimed step with every kernel traced (the timed steps trace "
                         "the GEMMs only)") if args.trace == "gemm" else "the timed steps",
        "configs": configs,
        "pack": pack,
        "attention": att,
        "device": device_info(dev, sclk),
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
