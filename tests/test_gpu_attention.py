"""GPU parity of the attention entry points (reels_hip_attention_fwd / _bwd) against the f64
oracle (oracle.attention_forward / attention_backward, the exact math of
memory_efficient_attention, src/layers/attention.jl:106-221) on the same seeded bf16 / f16
inputs, through the host mirror reels_amd.memory_efficient_attention(_backward).

Tolerance: the scores, the softmax and every sum run in f32; the output, P (for the P V
product), dS and the gradients are rounded to the 16-bit type, so the bar is the bf16 bar of the
rest of the suite for the output (tests/_util.assert_parity: normwise and elementwise 1e-2). The
gradients carry one more 16-bit rounding, of dS before the dK and dQ products, and each query's
dS sums to zero over its keys, so an element of dK or dQ can be small next to the terms it sums:
3e-2 there (the reference rounds dk and dv to the element type after every query block, a
coarser scheme). A wrong index or a missing term gives errors of order one. The log-sum-exp is
f32 from exact 16-bit products: absolute 1e-4. Covered: ragged query and key counts (not multiples of the 128-query
and 64-key tiles), head dims 64 and 128, masks, causal, cross-attention shapes (few keys, many
queries), batches, f16, queries with no visible key, no keys at all, and a larger case checked
on a subset of queries; at head dim 128 both dK / dV kernels (64- and 256-key workgroups)."""
import numpy as np
import pytest

import oracle
from tests._util import assert_parity, bf16_bits, to_dev

pytestmark = pytest.mark.gpu
GTOL = 3e-2  # gradients


def _inputs(B, Sq, Sk, H, D, seed, dt="bf16"):
    rng = np.random.default_rng(seed)
    f = lambda *sh: rng.standard_normal(sh).astype(np.float32)
    q, k, v, dy = f(B, Sq, H, D), f(B, Sk, H, D), f(B, Sk, H, D), f(B, Sq, H, D)
    if dt == "bf16":
        return tuple(oracle.f32_to_bf16(a) for a in (q, k, v, dy))
    if dt == "f32":
        return q, k, v, dy
    return tuple(a.astype(np.float16).view(np.uint16) for a in (q, k, v, dy))


def _dev(a, d, dt):
    import torch
    if dt == "f32":
        return torch.from_numpy(a).to(d)
    t = to_dev(a, d)  # bf16 view of the bits
    return t if dt == "bf16" else t.view(torch.float16)


def _bits(t):
    import torch
    if t.dtype == torch.float32:
        return t.cpu().numpy()
    return bf16_bits(t.view(torch.bfloat16) if t.dtype == torch.float16 else t)


def _vals(bits, dt):
    if dt == "f32":
        return bits
    return oracle.bf16_to_f32(bits) if dt == "bf16" else bits.view(np.float16).astype(np.float32)


def _run(B, Sq, Sk, H, D, causal=False, mask=None, dt="bf16", seed=0, backward=True):
    import torch
    from reels_amd import memory_efficient_attention, memory_efficient_attention_backward
    d = torch.device("cuda:0")
    q, k, v, dy = _inputs(B, Sq, Sk, H, D, seed, dt)
    print(f"[case] attention B={B} Sq={Sq} Sk={Sk} H={H} D={D} causal={causal} "
          f"mask={mask is not None} {dt} seed={seed}", flush=True)
    tq, tk, tv, tdy = (_dev(a, d, dt) for a in (q, k, v, dy))
    res = memory_efficient_attention(tq, tk, tv, mask=None if mask is None else torch.from_numpy(mask),
                                     causal=causal)
    torch.cuda.synchronize()
    out = _vals(_bits(res.output), dt)
    lse = res.cache.logsumexp.cpu().numpy()
    elt = dt
    ro, rl = oracle.attention_forward(q, k, v, mask=mask, causal=causal, elt=elt)
    grads = None
    if backward:
        g = memory_efficient_attention_backward(tq, tk, tv, tdy, res.cache)
        torch.cuda.synchronize()
        grads = tuple(_vals(_bits(x), dt) for x in g)
        ref = oracle.attention_backward(q, k, v, dy, mask=mask, causal=causal, elt=elt)
        grads = (grads, ref)
    return out, lse, ro, rl, grads


def _check_fwd(out, lse, ro, rl, what, rows=None):
    if rows is not None:
        out, ro = out[:, rows], ro[:, rows]
        lse, rl = lse[:, :, rows], rl[:, :, rows]
    assert_parity(out, ro, f"{what} out")
    assert np.max(np.abs(lse - rl)) <= 1e-4, f"{what} lse: {np.max(np.abs(lse - rl)):.3e}"


def _check_bwd(grads, what):
    (dq, dk, dv), (rq, rk, rv) = grads
    assert_parity(dq, rq, f"{what} dq", tol=GTOL)
    assert_parity(dk, rk, f"{what} dk", tol=GTOL)
    assert_parity(dv, rv, f"{what} dv", tol=GTOL)


CASES = [
    # B, Sq, Sk, H, D, causal, masked, dtype
    (1, 200, 300, 2, 128, False, False, "bf16"),
    (2, 130, 70, 3, 64, False, True, "bf16"),
    (1, 256, 256, 2, 128, True, False, "bf16"),
    (1, 300, 300, 1, 64, True, False, "bf16"),
    (1, 77, 512, 2, 128, False, False, "f16"),   # cross-attention: text keys
    (1, 390, 257, 2, 128, False, False, "bf16"), # image keys (I2V cross-attention, 257 tokens)
    (1, 1, 5, 1, 64, False, False, "bf16"),
    (3, 65, 129, 2, 128, False, True, "f16"),
    (2, 100, 300, 2, 64, True, False, "f16"),    # causal with more keys than queries, batch 2
    (2, 129, 129, 3, 128, True, True, "bf16"),   # mask and causal together
    (1, 40, 200, 2, 128, False, False, "bf16"),  # one query step (dK / dV ring prologue only)
    (2, 192, 385, 1, 128, False, False, "f16"),  # whole query steps, keys one past 3 x 128
]


@pytest.mark.parametrize("B,Sq,Sk,H,D,causal,masked,dt", CASES)
def test_attention_parity(dev, B, Sq, Sk, H, D, causal, masked, dt):
    mask = None
    if masked:
        rng = np.random.default_rng(100 + Sq)
        mask = rng.random((Sq, Sk)) < 0.7
        mask[:, 0] = True  # every query sees at least one key
    out, lse, ro, rl, grads = _run(B, Sq, Sk, H, D, causal, mask, dt, seed=Sq + Sk)
    what = f"{B}x{Sq}x{Sk}x{H}x{D} causal={causal} masked={masked} {dt}"
    _check_fwd(out, lse, ro, rl, what)
    _check_bwd(grads, what)


# The head-dim-128 cases again through the dK / dV kernel with 256-key workgroups, which the
# launcher picks by grid size (for many keys); the environment
# variable REELS_HIP_ATTN_DKDV_KEYS fixes the choice. Added: causal with keys past every query
# (workgroups with no query step store zeros), and causal in f16.
WIDE = [c for c in CASES if c[4] == 128] + [(1, 100, 600, 2, 128, True, False, "bf16"),
                                            (1, 130, 300, 2, 128, True, False, "f16")]


@pytest.mark.parametrize("B,Sq,Sk,H,D,causal,masked,dt", WIDE)
def test_attention_parity_256_key_dkdv(dev, monkeypatch, B, Sq, Sk, H, D, causal, masked, dt):
    monkeypatch.setenv("REELS_HIP_ATTN_DKDV_KEYS", "256")
    test_attention_parity(dev, B, Sq, Sk, H, D, causal, masked, dt)


@pytest.mark.parametrize("D,dkdv_keys", [(64, None), (128, "256"), (128, "64")])
def test_attention_query_without_visible_key(dev, monkeypatch, D, dkdv_keys):
    # NaN output and lse for that query, as the reference; the other queries and the
    # gradients are unaffected (the query contributes nothing)
    if dkdv_keys:
        monkeypatch.setenv("REELS_HIP_ATTN_DKDV_KEYS", dkdv_keys)
    Sq, Sk = 70, 90
    mask = np.ones((Sq, Sk), bool)
    mask[5] = False
    out, lse, ro, rl, grads = _run(1, Sq, Sk, 2, D, mask=mask, seed=3)
    assert np.isnan(out[0, 5]).all() and np.isnan(lse[0, :, 5]).all()
    rows = [i for i in range(Sq) if i != 5]
    _check_fwd(out, lse, ro, rl, "no-visible-key rows", rows=rows)
    (dq, dk, dv), (rq, rk, rv) = grads
    assert np.all(dq[0, 5] == 0.0)
    assert_parity(dq[:, rows], rq[:, rows], "no-visible-key dq", tol=GTOL)
    assert_parity(dk, rk, "no-visible-key dk", tol=GTOL)
    assert_parity(dv, rv, "no-visible-key dv", tol=GTOL)


def test_attention_no_keys(dev):
    # Sk = 0: output 0/0 = NaN and lse -Inf + log(0) = -Inf (attention.jl:164-167 with no key
    # block); dk, dv are empty, dq zero
    import torch
    from reels_amd import memory_efficient_attention, memory_efficient_attention_backward
    q = torch.randn(1, 10, 2, 64, device=dev).to(torch.bfloat16)
    k = torch.zeros(1, 0, 2, 64, device=dev, dtype=torch.bfloat16)
    res = memory_efficient_attention(q, k, k)
    torch.cuda.synchronize()
    assert torch.isnan(res.output.float()).all()
    assert torch.isinf(res.cache.logsumexp).all() and (res.cache.logsumexp < 0).all()
    g = memory_efficient_attention_backward(q, k, k, torch.ones_like(q), res.cache)
    torch.cuda.synchronize()
    assert g.k.numel() == 0 and g.v.numel() == 0
    assert (g.q.float() == 0).all()


def test_attention_larger_subset(dev):
    # 2048 queries x 3000 keys x 4 heads, head dim 128: the whole output against the oracle on
    # every 17th query (queries are independent in the forward)
    import torch
    from reels_amd import memory_efficient_attention
    B, Sq, Sk, H, D = 1, 2048, 3000, 4, 128
    q, k, v, _ = _inputs(B, Sq, Sk, H, D, seed=9)
    print(f"[case] attention subset B={B} Sq={Sq} Sk={Sk} H={H} D={D}", flush=True)
    res = memory_efficient_attention(*(to_dev(a, dev) for a in (q, k, v)))
    torch.cuda.synchronize()
    rows = np.arange(0, Sq, 17)
    ro, rl = oracle.attention_forward(q[:, rows], k, v, elt="bf16")
    out = oracle.bf16_to_f32(bf16_bits(res.output))[:, rows]
    lse = res.cache.logsumexp.cpu().numpy()[:, :, rows]
    assert_parity(out, ro, "subset out")
    assert np.max(np.abs(lse - rl)) <= 1e-4


def test_attention_is_deterministic(dev):
    import torch
    from reels_amd import memory_efficient_attention, memory_efficient_attention_backward
    q, k, v, dy = (to_dev(a, dev) for a in _inputs(1, 300, 400, 2, 128, seed=11))
    outs = []
    for _ in range(2):
        r = memory_efficient_attention(q, k, v)
        g = memory_efficient_attention_backward(q, k, v, dy, r.cache)
        torch.cuda.synchronize()
        outs.append([r.output.clone(), r.cache.logsumexp.clone(), g.q.clone(), g.k.clone(), g.v.clone()])
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           b.view(torch.int16) if b.dtype == torch.bfloat16 else b)


def test_attention_argument_errors(dev):
    import torch
    from reels_amd import memory_efficient_attention
    q = torch.zeros(1, 4, 2, 64, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="head dimensions differ"):
        memory_efficient_attention(q, torch.zeros(1, 4, 2, 128, device=dev, dtype=torch.bfloat16), q)
    with pytest.raises(ValueError, match="tile sizes must be positive"):
        memory_efficient_attention(q, q, q, query_block=0)
    with pytest.raises(ValueError, match="mask shape differs"):
        memory_efficient_attention(q, q, q, mask=torch.ones(3, 4, dtype=torch.bool))
    with pytest.raises(ValueError, match="head_dim must be between 1 and 128"):
        x = torch.zeros(1, 4, 2, 160, device=dev, dtype=torch.bfloat16)
        memory_efficient_attention(x, x, x)
    with pytest.raises(TypeError, match="share one dtype"):
        x = torch.zeros(1, 4, 2, 64, device=dev, dtype=torch.float64)
        memory_efficient_attention(x, x, x)


def test_attention_wan14b_self_attention_full_size(dev):
    """The benchmarked shape: Wan-2.1-14B self-attention of one block, 1 x 32760 tokens x 40 heads
    x 128 (src/models/wan21/transformer.jl:199), bf16 ~N(0, 1). Against the f64 oracle: out, lse
    and dq of 6 sampled queries (the first and the last among them) in every head; dk and dv of
    6 sampled keys (the first and the last among them) in heads 0 and 39, whose oracle streams
    all 32760 queries (the dK / dV kernel accumulates over 512 query steps). Every gradient
    element: the exact identities dq, dk, dv (2 dy) = 2 (dq, dk, dv) (dy enters linearly and
    scaling by 2 commutes with every rounding)."""
    import torch
    from reels_amd import memory_efficient_attention, memory_efficient_attention_backward
    B, S, H, D = 1, 32760, 40, 128
    print(f"[case] attention full size B={B} S={S} H={H} D={D} bf16", flush=True)
    g = torch.Generator(device=dev).manual_seed(32760)
    q, k, v, dy = (torch.randn((B, S, H, D), generator=g, device=dev).to(torch.bfloat16)
                   for _ in range(4))
    res = memory_efficient_attention(q, k, v)
    gr = memory_efficient_attention_backward(q, k, v, dy, res.cache)
    gr2 = memory_efficient_attention_backward(q, k, v, dy * 2, res.cache)
    torch.cuda.synchronize()
    for a, b2, name in zip(gr, gr2, ("dq", "dk", "dv")):
        assert torch.equal((a * 2).view(torch.int16), b2.view(torch.int16)), f"{name}(2dy) != 2 {name}"
    del gr2
    host = [bf16_bits(t) for t in (q, k, v, dy)]
    out = oracle.bf16_to_f32(bf16_bits(res.output))
    lse = res.cache.logsumexp.cpu().numpy()
    dq, dk, dv = (oracle.bf16_to_f32(bf16_bits(t)) for t in gr)
    rng = np.random.default_rng(5)
    qr = np.unique(np.concatenate([[0, S - 1], rng.integers(1, S - 1, 4)]))
    got = {n: [] for n in ("out", "lse", "dq", "dk", "dv")}
    ref = {n: [] for n in got}
    for h in range(H):
        r = oracle.attention_sampled(*host, 0, h, qrows=qr)
        got["out"].append(out[0, qr, h]); ref["out"].append(r["out"])
        got["lse"].append(lse[0, h, qr]); ref["lse"].append(r["lse"])
        got["dq"].append(dq[0, qr, h]); ref["dq"].append(r["dq"])
    kc = np.unique(np.concatenate([[0, S - 1], rng.integers(1, S - 1, 4)]))
    for h in (0, H - 1):
        print(f"[case] attention full size: oracle dk/dv of head {h}", flush=True)
        r = oracle.attention_sampled(*host, 0, h, kcols=kc)
        got["dk"].append(dk[0, kc, h]); ref["dk"].append(r["dk"])
        got["dv"].append(dv[0, kc, h]); ref["dv"].append(r["dv"])
    cat = lambda xs: np.concatenate([np.ravel(x) for x in xs])
    assert_parity(cat(got["out"]), cat(ref["out"]), "full-size out")
    assert np.max(np.abs(cat(got["lse"]) - cat(ref["lse"]))) <= 1e-4
    for n in ("dq", "dk", "dv"):
        assert_parity(cat(got[n]), cat(ref[n]), f"full-size {n}", tol=GTOL)


# f32 tensors and head dims other than 64 / 128 run on the generic kernels (attention_g.hip):
# every product and sum in f32 with the probabilities unrounded, so f32 results meet an f32 bar
# (normwise 1e-5 against the f64 oracle, lse 1e-5) and 16-bit results the bars of the tuned
# kernels above (the correction sum(dy .* out) reads the rounded output, as the reference's).
GENERIC = [
    # B, Sq, Sk, H, D, causal, masked, dtype
    (1, 200, 300, 2, 128, False, False, "f32"),
    (2, 130, 70, 3, 64, True, True, "f32"),
    (1, 77, 512, 2, 40, False, False, "f32"),    # UMT5-like head dim, text keys
    (1, 97, 129, 2, 80, True, False, "bf16"),
    (2, 65, 100, 1, 100, False, True, "f16"),
    (1, 33, 47, 3, 32, False, False, "bf16"),
    (1, 1, 5, 1, 7, False, False, "f32"),        # odd head dim, one query
]


@pytest.mark.parametrize("B,Sq,Sk,H,D,causal,masked,dt", GENERIC)
def test_attention_generic_parity(dev, B, Sq, Sk, H, D, causal, masked, dt):
    mask = None
    if masked:
        rng = np.random.default_rng(200 + Sq)
        mask = rng.random((Sq, Sk)) < 0.7
        mask[:, 0] = True
    out, lse, ro, rl, grads = _run(B, Sq, Sk, H, D, causal, mask, dt, seed=Sq * 3 + Sk)
    what = f"generic {B}x{Sq}x{Sk}x{H}x{D} causal={causal} masked={masked} {dt}"
    if dt == "f32":
        assert_parity(out, ro, f"{what} out", tol=1e-5)
        assert np.max(np.abs(lse - rl)) <= 1e-5, f"{what} lse: {np.max(np.abs(lse - rl)):.3e}"
        (dq, dk, dv), (rq, rk, rv) = grads
        for name, a, r in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
            assert_parity(a, r, f"{what} {name}", tol=1e-5)
    else:
        _check_fwd(out, lse, ro, rl, what)
        _check_bwd(grads, what)


def test_attention_generic_no_visible_key_and_no_keys(dev):
    """The generic kernels' edge cases: a query that sees no key gets NaN output and lse and adds
    nothing to the gradients; without keys the output is NaN, lse -Inf and dk, dv are empty."""
    import torch
    from reels_amd import memory_efficient_attention, memory_efficient_attention_backward
    Sq, Sk = 20, 33
    mask = np.ones((Sq, Sk), bool)
    mask[5] = False
    out, lse, ro, rl, grads = _run(1, Sq, Sk, 2, 48, mask=mask, dt="f32", seed=9)
    assert np.isnan(out[0, 5]).all() and np.isnan(lse[0, :, 5]).all()
    keep = np.arange(Sq) != 5
    assert_parity(out[:, keep], ro[:, keep], "no-key query: other outputs", tol=1e-5)
    (dq, dk, dv), (rq, rk, rv) = grads
    assert np.all(dq[0, 5] == 0)
    assert_parity(dk, rk, "no-key query: dk", tol=1e-5)
    d = torch.device("cuda:0")
    q = torch.randn(1, 4, 1, 24, device=d)
    kk = torch.zeros(1, 0, 1, 24, device=d)
    res = memory_efficient_attention(q, kk, kk)
    torch.cuda.synchronize()
    assert torch.isnan(res.output).all() and torch.isneginf(res.cache.logsumexp).all()
