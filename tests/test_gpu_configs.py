"""GPU parity on the remaining BASELINE workloads:
  * cross-attention K/V projections 5120->5120 with 77 / 333 / 512 text tokens (skinny M);
  * Wan-2.1-1.3B projections at 32760 tokens (q/k/v/o 1536^2, ffn 1536<->8960; sampled rows
    against the oracle, exact doubling identities over the whole output);
  * the 1.3B linear stack chained through gelu_tanh (q -> k -> v -> o -> ffn.0 -> GELU -> ffn.2),
    two layers at 128 tokens: every linear's forward and backward checked against the oracle
    on the GPU's own intermediates, and the end-to-end drift against an all-oracle chain.
Tolerances as tests/_util.assert_parity (bf16 bar 1e-2); end-to-end drift 3e-2."""
import numpy as np
import pytest

import oracle
from tests._util import assert_parity, bf16_bits, bf16_f32, to_dev

pytestmark = pytest.mark.gpu


def _weights(seed, N, K, r):
    w = oracle.normal_bf16(seed, (N, K), 0.02)
    q, s, st = oracle.pack(w, "bf16")
    assert st == 0
    A = oracle.normal_bf16(seed + 1, (K, r), 0.01)
    B = oracle.normal_bf16(seed + 2, (r, N), 0.01)
    return q, s, A, B


def _dev_layer(dev, q, s, A, B):
    from reels_amd import QuantizedMatrix
    return QuantizedMatrix(to_dev(q, dev, "raw"), to_dev(s, dev, "raw")), to_dev(A, dev), to_dev(B, dev)


@pytest.mark.parametrize("M", [77, 333, 512])
def test_cross_attention_skinny_tokens(dev, M):
    import torch
    from reels_amd import i8lora_backward, i8lora_forward
    K = N = 5120
    r, c = 32, 1.0
    q, s, A, B = _weights(900 + M, N, K, r)
    x = oracle.normal_bf16(910 + M, (M, K), 1.0)
    dy = oracle.normal_bf16(920 + M, (M, N), 1.0)
    print(f"[configs] cross-attn M={M}", flush=True)
    W, Ad, Bd = _dev_layer(dev, q, s, A, B)
    y, h = i8lora_forward(to_dev(x, dev), W, Ad, Bd, None, c, save_h=True)
    dx, dA, dB = i8lora_backward(to_dev(dy, dev), to_dev(x, dev), W, Ad, Bd, c, h=h)
    torch.cuda.synchronize(dev)
    rows = np.unique(np.concatenate([np.arange(0, M, max(1, M // 40)), np.arange(max(0, M - 8), M)]))
    yo, _ = oracle.lora_forward(x, q, s, A, B, c, rows=rows)
    go = oracle.lora_backward(dy, x, q, s, A, B, c, rows=rows)
    assert_parity(bf16_f32(y)[rows], yo, f"cross-attn M={M} y")
    assert_parity(bf16_f32(dx)[rows], go["dx"], f"cross-attn M={M} dx")
    assert_parity(dA.cpu().numpy(), go["dA"], f"cross-attn M={M} dA")
    assert_parity(dB.cpu().numpy(), go["dB"], f"cross-attn M={M} dB")


@pytest.mark.parametrize("K,N", [(1536, 1536), (1536, 8960), (8960, 1536)])
def test_wan13b_projections_full_tokens(dev, K, N):
    import torch
    from reels_amd import i8lora_backward, i8lora_forward
    M, r, c = 32760, 32, 1.0
    q, s, A, B = _weights(1000 + K + N, N, K, r)
    x = oracle.normal_bf16(1010 + K, (M, K), 1.0)
    dy = oracle.normal_bf16(1020 + N, (M, N), 1.0)
    print(f"[configs] wan1.3b M={M} K={K} N={N}", flush=True)
    W, Ad, Bd = _dev_layer(dev, q, s, A, B)
    xd, dyd = to_dev(x, dev), to_dev(dy, dev)
    y, h = i8lora_forward(xd, W, Ad, Bd, None, c, save_h=True)
    dx, dA, dB = i8lora_backward(dyd, xd, W, Ad, Bd, c, h=h)
    y2, _ = i8lora_forward(xd * 2, W, Ad, Bd, None, c)
    dx2, dA2, dB2 = i8lora_backward(dyd * 2, xd, W, Ad, Bd, c, h=h)
    torch.cuda.synchronize(dev)
    assert torch.equal(y2, y * 2) and torch.equal(dx2, dx * 2)
    assert torch.equal(dA2, dA * 2) and torch.equal(dB2, dB * 2)
    rng = np.random.default_rng(K + N)
    rows = np.concatenate([rng.choice(M - 32, 24, replace=False), np.arange(M - 8, M)])
    kc = rng.choice(K, 32, replace=False)
    nc = rng.choice(N, 32, replace=False)
    yo, _ = oracle.lora_forward(x, q, s, A, B, c, rows=rows)
    go = oracle.lora_backward(dy, x, q, s, A, B, c, rows=rows, kcols=kc, ncols=nc)
    assert_parity(bf16_f32(y)[rows], yo, f"1.3B {K}x{N} y")
    assert_parity(bf16_f32(dx)[rows], go["dx"], f"1.3B {K}x{N} dx")
    assert_parity(dA.cpu().numpy()[kc], go["dA"], f"1.3B {K}x{N} dA")
    assert_parity(dB.cpu().numpy()[:, nc], go["dB"], f"1.3B {K}x{N} dB")


def test_wan13b_chain_with_gelu(dev):
    import torch
    from reels_amd import gelu_tanh, gelu_tanh_backward, i8lora_backward, i8lora_forward
    M, D, F, r, c, layers = 128, 1536, 8960, 32, 1.0, 2
    shapes = [("q", D, D), ("k", D, D), ("v", D, D), ("o", D, D), ("ffn0", D, F), ("ffn2", F, D)]
    params = []
    for li in range(layers):
        for j, (name, K, N) in enumerate(shapes):
            params.append((f"{li}.{name}", K, N) + _weights(2000 + 10 * (6 * li + j), N, K, r))
    x0 = oracle.normal_bf16(2999, (M, D), 1.0)
    print("[configs] 1.3B chain, 2 layers x (q,k,v,o,ffn.0,gelu,ffn.2), M=128", flush=True)

    # ---- forward on the GPU, keeping every intermediate
    acts, hs, pre_gelu = [x0], [], {}
    cur = to_dev(x0, dev)
    dev_params = []
    for (name, K, N, q, s, A, B) in params:
        W, Ad, Bd = _dev_layer(dev, q, s, A, B)
        dev_params.append((W, Ad, Bd))
        y, h = i8lora_forward(cur, W, Ad, Bd, None, c, save_h=True)
        hs.append(h)
        if name.endswith("ffn0"):
            pre_gelu[name] = y
            y = gelu_tanh(y)
        cur = y
        acts.append(bf16_bits(y))
    torch.cuda.synchronize(dev)

    # per-linear forward parity on the GPU's own inputs
    inputs = []
    xin = x0
    for i, (name, K, N, q, s, A, B) in enumerate(params):
        inputs.append(xin)
        yo, _ = oracle.lora_forward(xin, q, s, A, B, c)
        got = pre_gelu[name] if name.endswith("ffn0") else None
        if got is not None:
            assert_parity(bf16_f32(got), yo, f"chain {name} y")
            assert np.array_equal(acts[i + 1], bf16_bits(gelu_tanh(got)))
        else:
            assert_parity(oracle.bf16_to_f32(acts[i + 1]), yo, f"chain {name} y")
        xin = acts[i + 1]

    # end-to-end drift against a chain computed in f64 from the weights the path multiplies. At
    # 128 tokens the few-token path (at most 240 tokens here) multiplies the exact int8 codes and
    # applies s to the f32 sum, so the model is the exact-weight chain (f64 q s); with more
    # tokens the path multiplies the bf16 dequantization wd = bf16(fl32(q s)) (oracle.dequant
    # "bf16"). h = bf16(x A), bf16 between layers in both. The drift against the other model is
    # printed beside it; the per-linear checks above bound each layer's error.
    def deq_forward(xb, q, s, A, B):
        f64 = lambda bits: oracle.bf16_to_f32(bits).astype(np.float64)
        xf = f64(xb)
        h = f64(oracle.f32_to_bf16((xf @ f64(A)).astype(np.float32)))
        return xf @ f64(oracle.dequant(q, s, "bf16")).T + c * (h @ f64(B))
    xo, xe = x0, x0
    for (name, K, N, q, s, A, B) in params:
        yb = oracle.f32_to_bf16(deq_forward(xo, q, s, A, B).astype(np.float32))
        xo = oracle.gelu_tanh(yb) if name.endswith("ffn0") else yb
        ye, _ = oracle.lora_forward(xe, q, s, A, B, c)
        yeb = oracle.f32_to_bf16(ye.astype(np.float32))
        xe = oracle.gelu_tanh(yeb) if name.endswith("ffn0") else yeb
    got = oracle.bf16_to_f32(acts[-1]).astype(np.float64)
    for label, ref in (("exact-weight", xe), ("bf16-dequantized", xo)):
        rf = oracle.bf16_to_f32(ref).astype(np.float64)
        print(f"[configs] chain drift vs the {label} f64 chain: normwise "
              f"{np.abs(got - rf).max() / np.abs(rf).max():.3e}", flush=True)
    model = xe if M <= 240 else xo
    assert_parity(got, oracle.bf16_to_f32(model), "chain output drift", tol=3e-2)

    # ---- backward on the GPU, layer by layer, each checked against the oracle on its inputs
    g = oracle.normal_bf16(3999, (M, D), 1.0)
    gd = to_dev(g, dev)
    for i in reversed(range(len(params))):
        name, K, N, q, s, A, B = params[i]
        W, Ad, Bd = dev_params[i]
        if name.endswith("ffn0"):
            gd = gelu_tanh_backward(pre_gelu[name], gd)
        dyb = bf16_bits(gd)
        dx, dA, dB = i8lora_backward(gd, to_dev(inputs[i], dev), W, Ad, Bd, c, h=hs[i])
        torch.cuda.synchronize(dev)
        go = oracle.lora_backward(dyb, inputs[i], q, s, A, B, c)
        assert_parity(bf16_f32(dx), go["dx"], f"chain {name} dx")
        assert_parity(dA.cpu().numpy(), go["dA"], f"chain {name} dA")
        assert_parity(dB.cpu().numpy(), go["dB"], f"chain {name} dB")
        gd = dx


def test_wan13b_30_layer_chain_at_full_tokens(dev):
    """Config 4 at its configured size: 30 Wan-2.1-1.3B layers, each q -> k -> v -> o -> ffn.0 ->
    gelu_tanh -> ffn.2 (dim 1536, ffn 8960; src/models/wan21/transformer.jl:289-292,
    src/layers/linear.jl:61-68), 32760 tokens, LoRA r = 32 on all 180 linears, one forward then
    one backward (dX chained back through the GELU pullback, dA and dB for every linear).
    Every linear is checked on the GPU's own inputs: sampled rows of y and of dx (including the
    last token) against the oracle; dA and dB on sampled columns for all six linears of the first
    layer (the end of the backward chain) and of the last layer (its start); the exact doubling
    identities y(2x) = 2 y(x) and dx(2dy) = 2 dx(dy), dA(2dy) = 2 dA, dB(2dy) = 2 dB for those
    twelve linears."""
    import time

    import torch
    from reels_amd import (gelu_tanh, gelu_tanh_backward, i8lora_backward, i8lora_forward,
                           quantize_frozen_matrix)
    M, D, F, r, c, layers = 32760, 1536, 8960, 32, 1.0, 30
    shapes = [("q", D, D), ("k", D, D), ("v", D, D), ("o", D, D), ("ffn0", D, F), ("ffn2", F, D)]
    g = torch.Generator(device=dev).manual_seed(4321)
    t0 = time.time()
    params = []
    for li in range(layers):
        for (name, K, N) in shapes:
            w = (torch.randn((N, K), generator=g, device=dev) * 0.02).to(torch.bfloat16)
            W = quantize_frozen_matrix(w, torch.bfloat16)
            A = (torch.randn((K, r), generator=g, device=dev) * 0.01).to(torch.bfloat16)
            B = (torch.randn((r, N), generator=g, device=dev) * 0.01).to(torch.bfloat16)
            params.append((f"{li}.{name}", K, N, W, A, B))
    x0 = torch.randn((M, D), generator=g, device=dev).to(torch.bfloat16)
    gout = torch.randn((M, D), generator=g, device=dev).to(torch.bfloat16)
    print(f"[configs] cfg4 chain: {layers} layers x 6 linears, M={M}", flush=True)

    # forward, keeping each linear's input, h and (ffn.0) the pre-GELU output
    inputs, hs, outs, pre = [], [], [], {}
    cur = x0
    for (name, K, N, W, A, B) in params:
        inputs.append(cur)
        y, h = i8lora_forward(cur, W, A, B, None, c, save_h=True)
        hs.append(h)
        outs.append(y)
        if name.endswith("ffn0"):
            pre[name] = y
            y = gelu_tanh(y)
        cur = y
    # backward
    dys, dxs, grads = [None] * len(params), [None] * len(params), [None] * len(params)
    gd = gout
    for i in reversed(range(len(params))):
        name, K, N, W, A, B = params[i]
        if name.endswith("ffn0"):
            gd = gelu_tanh_backward(pre[name], gd)
        dys[i] = gd
        dx, dA, dB = i8lora_backward(gd, inputs[i], W, A, B, c, h=hs[i])
        dxs[i], grads[i] = dx, (dA, dB)
        gd = dx
    torch.cuda.synchronize(dev)
    print(f"[configs] cfg4 chain ran on the GPU ({time.time() - t0:.1f} s with set-up)", flush=True)
    assert all(torch.isfinite(t).all() for t in (cur, gd))

    rng = np.random.default_rng(44)
    rows = np.concatenate([rng.choice(M - 1, 7, replace=False), [M - 1]])
    rt = torch.from_numpy(rows).to(dev)
    for i, (name, K, N, W, A, B) in enumerate(params):
        q, s = W.values.cpu().numpy(), W.scales.cpu().numpy()
        Ah, Bh = bf16_bits(A), bf16_bits(B)
        xr, dyr = bf16_bits(inputs[i][rt]), bf16_bits(dys[i][rt])
        yo, _ = oracle.lora_forward(xr, q, s, Ah, Bh, c)
        assert_parity(bf16_f32(outs[i][rt]), yo, f"cfg4 {name} y (sampled rows)")
        dxo = oracle.lora_backward(dyr, xr, q, s, Ah, Bh, c, want=("dx",))["dx"]
        assert_parity(bf16_f32(dxs[i][rt]), dxo, f"cfg4 {name} dx (sampled rows)")
        if i < len(shapes) or i >= len(params) - len(shapes):
            # the first layer (end of the backward chain) and the last (its start): dA, dB over
            # all tokens on sampled columns, and the doubling identities
            kc = rng.choice(K, 24, replace=False)
            nc = rng.choice(N, 24, replace=False)
            go = oracle.lora_backward(bf16_bits(dys[i]), bf16_bits(inputs[i]), q, s, Ah, Bh, c,
                                      rows=rows[:1], kcols=kc, ncols=nc, want=("dA", "dB"))
            dA, dB = grads[i]
            assert_parity(dA.cpu().numpy()[kc], go["dA"], f"cfg4 {name} dA (sampled k)")
            assert_parity(dB.cpu().numpy()[:, nc], go["dB"], f"cfg4 {name} dB (sampled n)")
            y2, _ = i8lora_forward(inputs[i] * 2, W, A, B, None, c)
            dx2, dA2, dB2 = i8lora_backward(dys[i] * 2, inputs[i], W, A, B, c, h=hs[i])
            torch.cuda.synchronize(dev)
            assert torch.equal(y2, outs[i] * 2) and torch.equal(dx2, dxs[i] * 2)
            assert torch.equal(dA2, dA * 2) and torch.equal(dB2, dB * 2)
    print(f"[configs] cfg4 chain checked ({time.time() - t0:.1f} s)", flush=True)
