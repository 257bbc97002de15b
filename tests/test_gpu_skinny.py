"""The few-token path's single launch (reels_amd/csrc/skinny.hip): output tiles wait for the
adapter's rank projection l, published by the adapter blocks of the same launch, and a tile that
stops waiting computes l itself with the adapter blocks' code and order. With split tiles the
counters live in the call's own workspace, cleared by a one-block kernel just before the launch;
row-wave launches (a few hundred tokens on a large weight) hand l and the adapter tiles' split
partials over under a key of the launch (its dispatch in its queue and the host call's nonce)
and clear nothing.

These tests force the fallback from the host (REELS_HIP_SKINNY_SPIN=0: no wait at all, so
split-0 adapter blocks also compute the other splits' partials) and require the same bits as
the normal run; run calls concurrently on many streams, HIP graphs of few-token calls captured
on one stream and replayed at the same time on two streams, graphs replayed on changing inputs,
row-wave calls on workspaces of any contents, and repeat calls. The parity of the values themselves against the oracle is in
tests/test_gpu_configs.py (cross-attention shapes) and tests/test_gpu_lora.py."""
import numpy as np
import pytest

import oracle
from tests._util import assert_parity, bf16_f32, to_dev

pytestmark = pytest.mark.gpu


def _case(dev, M, K, N, r, seed, elt="bf16"):
    import torch
    from reels_amd import QuantizedMatrix
    w = oracle.normal_bf16(seed, (N, K), 0.02)
    q, s, st = oracle.pack(w, "bf16")
    assert st == 0
    x = oracle.normal_bf16(seed + 1, (M, K), 1.0)
    A = oracle.normal_bf16(seed + 2, (K, r), 0.01)
    B = oracle.normal_bf16(seed + 3, (r, N), 0.01)
    dy = oracle.normal_bf16(seed + 4, (M, N), 1.0)
    host = dict(x=x, q=q, s=s, A=A, B=B, dy=dy)
    if elt == "bf16":
        W = QuantizedMatrix(to_dev(q, dev, "raw"), to_dev(s, dev, "raw"))
        put = lambda a: to_dev(a, dev)
    else:
        W = QuantizedMatrix(to_dev(q, dev, "raw"), to_dev(s, dev, "raw"), torch.float16)
        put = lambda a: torch.from_numpy(oracle.bf16_to_f32(a)).to(torch.float16).to(dev)
    devs = dict(x=put(x), A=put(A), B=put(B), dy=put(dy), W=W)
    return host, devs


def _run(d, c):
    from reels_amd import i8lora_backward, i8lora_forward
    y, h = i8lora_forward(d["x"], d["W"], d["A"], d["B"], None, c, save_h=True)
    dx, dA, dB = i8lora_backward(d["dy"], d["x"], d["W"], d["A"], d["B"], c, h=None)
    return y, h, dx, dA, dB


@pytest.mark.parametrize("M,K,N,r", [(77, 5120, 5120, 32), (100, 1536, 1536, 24), (200, 1536, 1024, 8)])
def test_output_tiles_computing_l_themselves_give_the_same_bits(dev, monkeypatch, M, K, N, r):
    import torch
    host, d = _case(dev, M, K, N, r, 4100 + M)
    c = 2.0
    print(f"[skinny] fallback M={M} K={K} N={N} r={r}", flush=True)
    ref = _run(d, c)
    torch.cuda.synchronize(dev)
    monkeypatch.setenv("REELS_HIP_SKINNY_SPIN", "0")
    for _ in range(2):
        got = _run(d, c)
        torch.cuda.synchronize(dev)
        for name, a, b in zip(("y", "h", "dx", "dA", "dB"), ref, got):
            assert torch.equal(a, b), f"{name} differs when output tiles compute l themselves"
    monkeypatch.delenv("REELS_HIP_SKINNY_SPIN")
    again = _run(d, c)
    torch.cuda.synchronize(dev)
    assert all(torch.equal(a, b) for a, b in zip(ref, again))
    rows = np.arange(0, M, 7)
    yo, ho = oracle.lora_forward(host["x"], host["q"], host["s"], host["A"], host["B"], c, rows=rows)
    assert_parity(bf16_f32(got[0])[rows], yo, f"fallback M={M} y")


def test_concurrent_streams(dev):
    """Calls on 70 streams at once: every result equals the same call made alone on the default
    stream."""
    import torch
    from reels_amd import i8lora_forward
    M, K, N, r, c = 77, 1536, 1536, 16, 1.0
    cases = [_case(dev, M, K, N, r, 4300 + 10 * i)[1] for i in range(4)]
    print("[skinny] 70 streams", flush=True)
    ref = []
    for d in cases:
        y, h = i8lora_forward(d["x"], d["W"], d["A"], d["B"], None, c, save_h=True)
        ref.append((y, h))
    torch.cuda.synchronize(dev)
    streams = [torch.cuda.Stream(device=dev) for _ in range(70)]
    outs = []
    for rep in range(2):
        for i, st in enumerate(streams):
            d = cases[i % len(cases)]
            st.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(st):
                outs.append((i % len(cases), *i8lora_forward(d["x"], d["W"], d["A"], d["B"], None, c,
                                                            save_h=True)))
    torch.cuda.synchronize(dev)
    for k, y, h in outs:
        assert torch.equal(y, ref[k][0]) and torch.equal(h, ref[k][1])


def test_graphs_captured_on_one_stream_replayed_concurrently(dev):
    """Few-token forwards and backwards captured into two HIP graphs on the same capture stream
    (torch.cuda.graph uses one side stream for every capture), then replayed at the same time on
    two streams, several rounds with eager work and synchronisations between them: each replay
    equals the eager call bit for bit. Counters kept per caller stream would be shared by the two
    graphs here."""
    import torch
    M, K, N, r, c = 77, 5120, 5120, 32, 1.0
    cases = [_case(dev, M, K, N, r, 4700 + 10 * i)[1] for i in range(2)]
    print("[skinny] two graphs replayed concurrently", flush=True)
    eager = [_run(d, c) for d in cases]
    torch.cuda.synchronize(dev)
    for d in cases:  # warm-up on a side stream (first-call set-up stays out of the captures)
        s = torch.cuda.Stream(device=dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(s):
            _run(d, c)
        torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize(dev)
    graphs, outs = [], []
    for d in cases:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs.append(_run(d, c))
        graphs.append(g)
    torch.cuda.synchronize(dev)
    streams = [torch.cuda.Stream(device=dev) for _ in graphs]
    for rnd in range(4):
        for g, st in zip(graphs, streams):
            st.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(st):
                g.replay()
        for st in streams:
            torch.cuda.current_stream(dev).wait_stream(st)
        torch.cuda.synchronize(dev)
        for i, (got, ref) in enumerate(zip(outs, eager)):
            for name, a, b in zip(("y", "h", "dx", "dA", "dB"), got, ref):
                assert torch.equal(a, b), f"round {rnd}: graph {i} {name} differs from eager"
        _run(cases[rnd % 2], c)  # eager work between the rounds
        torch.cuda.synchronize(dev)


def test_f16_fallback_and_repeat(dev, monkeypatch):
    import torch
    host, d = _case(dev, 77, 1536, 1536, 32, 4500, "f16")
    c = 0.5
    print("[skinny] f16 fallback", flush=True)
    ref = _run(d, c)
    torch.cuda.synchronize(dev)
    monkeypatch.setenv("REELS_HIP_SKINNY_SPIN", "0")
    got = _run(d, c)
    torch.cuda.synchronize(dev)
    for name, a, b in zip(("y", "h", "dx", "dA", "dB"), ref, got):
        assert torch.equal(a, b), f"f16 {name} differs when output tiles compute l themselves"


@pytest.mark.parametrize("r", [3, 160])
def test_few_tokens_any_rank(dev, r):
    """Ranks that are not a multiple of 16 and ranks above 128 on the few-token path: several
    adapter row blocks (160 = 5 of 32) and rank chunks in the epilogue's l R product, padding past
    the rank. 77 tokens on 5120 x 5120; y, h, dx, dA, dB against the oracle, h recomputed for the
    backward equal to the saved one."""
    import torch
    from reels_amd import i8lora_backward, i8lora_forward
    M, K, N = 77, 5120, 5120
    host, d = _case(dev, M, K, N, r, 4600 + r)
    c = float(np.float32(r) / np.float32(r))
    print(f"[skinny] rank {r} at {M} tokens", flush=True)
    y, h = i8lora_forward(d["x"], d["W"], d["A"], d["B"], None, c, save_h=True)
    dx, dA, dB = i8lora_backward(d["dy"], d["x"], d["W"], d["A"], d["B"], c, h=h)
    dx2, dA2, dB2 = i8lora_backward(d["dy"], d["x"], d["W"], d["A"], d["B"], c, h=None)
    torch.cuda.synchronize(dev)
    assert torch.equal(dx, dx2) and torch.equal(dA, dA2) and torch.equal(dB, dB2)
    yo, ho = oracle.lora_forward(host["x"], host["q"], host["s"], host["A"], host["B"], c)
    go = oracle.lora_backward(host["dy"], host["x"], host["q"], host["s"], host["A"], host["B"], c)
    assert_parity(bf16_f32(y), yo, f"rank {r} y")
    assert_parity(bf16_f32(h), ho, f"rank {r} h")
    assert_parity(bf16_f32(dx), go["dx"], f"rank {r} dx")
    assert_parity(dA.cpu().numpy(), go["dA"], f"rank {r} dA")
    assert_parity(dB.cpu().numpy(), go["dB"], f"rank {r} dB")


def test_thousand_tokens_on_a_small_weight(dev):
    """Config 1's shape (one 1536 x 1536 linear, 1024 tokens, r 16, alpha 16): a small weight takes
    the few-token path up to 1024 tokens (13 token blocks); y, h, dx, dA, dB against the oracle."""
    import torch
    from reels_amd import i8lora_backward, i8lora_forward
    M, K, N, r = 1024, 1536, 1536, 16
    host, d = _case(dev, M, K, N, r, 4700)
    c = 1.0
    print("[skinny] 1024 tokens on 1536 x 1536", flush=True)
    y, h = i8lora_forward(d["x"], d["W"], d["A"], d["B"], None, c, save_h=True)
    dx, dA, dB = i8lora_backward(d["dy"], d["x"], d["W"], d["A"], d["B"], c, h=h)
    torch.cuda.synchronize(dev)
    yo, ho = oracle.lora_forward(host["x"], host["q"], host["s"], host["A"], host["B"], c)
    go = oracle.lora_backward(host["dy"], host["x"], host["q"], host["s"], host["A"], host["B"], c)
    assert_parity(bf16_f32(y), yo, "1024 tokens y")
    assert_parity(bf16_f32(h), ho, "1024 tokens h")
    assert_parity(bf16_f32(dx), go["dx"], "1024 tokens dx")
    assert_parity(dA.cpu().numpy(), go["dA"], "1024 tokens dA")
    assert_parity(dB.cpu().numpy(), go["dB"], "1024 tokens dB")


def test_row_wave_dx_over_a_long_reduction(dev):
    """dX on row-wave tiles over a reduction longer than the split tiles' scale table held: 200
    tokens on a 1536 -> 8960 weight (dX reduces over the 8960 outputs; the row-wave dX copies
    each step's 128 scales with its codes). y, h, dx, dA, dB against the oracle, and the same
    bits when repeated."""
    import torch
    from reels_amd import i8lora_backward, i8lora_forward
    M, K, N, r = 200, 1536, 8960, 32
    host, d = _case(dev, M, K, N, r, 4800)
    c = 1.0
    print("[skinny] row-wave dX, 200 tokens on 1536 -> 8960", flush=True)
    y, h = i8lora_forward(d["x"], d["W"], d["A"], d["B"], None, c, save_h=True)
    dx, dA, dB = i8lora_backward(d["dy"], d["x"], d["W"], d["A"], d["B"], c, h=h)
    dx2, _, _ = i8lora_backward(d["dy"], d["x"], d["W"], d["A"], d["B"], c, h=h)
    torch.cuda.synchronize()
    assert torch.equal(dx, dx2)
    yo, ho = oracle.lora_forward(host["x"], host["q"], host["s"], host["A"], host["B"], c)
    go = oracle.lora_backward(host["dy"], host["x"], host["q"], host["s"], host["A"], host["B"], c)
    assert_parity(bf16_f32(y), yo, "long-reduction y")
    assert_parity(bf16_f32(h), ho, "long-reduction h")
    assert_parity(bf16_f32(dx), go["dx"], "long-reduction dx")
    assert_parity(dA.cpu().numpy(), go["dA"], "long-reduction dA")
    assert_parity(dB.cpu().numpy(), go["dB"], "long-reduction dB")


@pytest.mark.parametrize("M,K,N,r", [(512, 1536, 1536, 32), (400, 1536, 1536, 16), (160, 1024, 4096, 8),
                                     (77, 1536, 1536, 32), (40, 1536, 1536, 32)])
def test_row_wave_tiles_on_narrow_weights(dev, M, K, N, r):
    """Row-wave tiles where 128-row tiles cannot fill the GPU. Tiles of 64 weight rows x 64
    tokens: a few hundred tokens on 1536 x 1536 (the 1.3B model's cross-attention K/V at 512
    text tokens) in both directions, 160 tokens on 1024 -> 4096 in the forward. Fewer tiles than
    CUs on reductions up to 4096 deep: the 4096-deep dX of that shape (80 tiles), 77 and 40
    tokens on 1536 x 1536 (72 and 48 tiles). y, h, dx, dA, dB against the oracle, and the same
    bits when repeated."""
    import torch
    from reels_amd import i8lora_backward, i8lora_forward
    host, d = _case(dev, M, K, N, r, 4900 + M)
    c = 2.0
    print(f"[skinny] 64 x 64 row-wave tiles M={M} K={K} N={N} r={r}", flush=True)
    y, h = i8lora_forward(d["x"], d["W"], d["A"], d["B"], None, c, save_h=True)
    dx, dA, dB = i8lora_backward(d["dy"], d["x"], d["W"], d["A"], d["B"], c, h=None)
    y2, _ = i8lora_forward(d["x"], d["W"], d["A"], d["B"], None, c, save_h=True)
    dx2, dA2, dB2 = i8lora_backward(d["dy"], d["x"], d["W"], d["A"], d["B"], c, h=None)
    torch.cuda.synchronize()
    assert torch.equal(y, y2) and torch.equal(dx, dx2) and torch.equal(dA, dA2) and torch.equal(dB, dB2)
    yo, ho = oracle.lora_forward(host["x"], host["q"], host["s"], host["A"], host["B"], c)
    go = oracle.lora_backward(host["dy"], host["x"], host["q"], host["s"], host["A"], host["B"], c)
    assert_parity(bf16_f32(y), yo, f"M={M} y")
    assert_parity(bf16_f32(h), ho, f"M={M} h")
    assert_parity(bf16_f32(dx), go["dx"], f"M={M} dx")
    assert_parity(dA.cpu().numpy(), go["dA"], f"M={M} dA")
    assert_parity(dB.cpu().numpy(), go["dB"], f"M={M} dB")

def _abi_calls(dev, M, K, N, r, c, ws):
    """Forward and backward through the C-ABI on an explicit workspace ws (uint8, large enough
    for both)."""
    import ctypes
    import torch
    from reels_amd import _lib
    L = _lib.lib()
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def run(d):
        bf = torch.bfloat16
        y, h = torch.empty((M, N), dtype=bf, device=dev), torch.empty((M, r), dtype=bf, device=dev)
        dx = torch.empty((M, K), dtype=bf, device=dev)
        dA = torch.empty((K, r), dtype=torch.float32, device=dev)
        dB = torch.empty((r, N), dtype=torch.float32, device=dev)
        q, s = p(d["W"].values), p(d["W"].scales)
        _lib.check("fwd", L.reels_hip_i8lora_fwd(p(d["x"]), q, s, p(d["A"]), p(d["B"]), None, M, K, N,
                                                 r, c, p(y), p(h), p(ws), ws.numel(), st))
        _lib.check("bwd", L.reels_hip_i8lora_bwd(p(d["dy"]), p(d["x"]), p(h), q, s, p(d["A"]), p(d["B"]),
                                                 M, K, N, r, c, p(dx), p(dA), p(dB), p(ws), ws.numel(), st))
        return y, h, dx, dA, dB
    return run


@pytest.mark.parametrize("M", [77, 333, 512])
def test_row_wave_results_do_not_depend_on_the_workspace_contents(dev, M):
    """5120 x 5120 at 77 / 333 / 512 tokens (row-wave forward and dX, adapter tiles split 5 / 2 /
    1 ways): the same bits on a workspace of zeros, of 0xff bytes, of random bytes, and on the
    workspace a call on other inputs has just used (its keys and l still there)."""
    import torch
    from reels_amd import _lib, workspace_bytes
    K = N = 5120
    r, c = 32, 1.0
    print(f"[skinny] workspace contents M={M}", flush=True)
    _, a = _case(dev, M, K, N, r, 5100 + M)
    _, b = _case(dev, M, K, N, r, 5200 + M)
    wsn = max(workspace_bytes(M, K, N, r, _lib.WS_FWD, torch.bfloat16),
              workspace_bytes(M, K, N, r, _lib.WS_BWD, torch.bfloat16))
    ws = torch.zeros(wsn, dtype=torch.uint8, device=dev)
    run = _abi_calls(dev, M, K, N, r, c, ws)
    ref = run(a)
    torch.cuda.synchronize(dev)
    gen = torch.Generator(device=dev).manual_seed(M)
    fills = [("0xff", lambda: ws.fill_(255)),
             ("random", lambda: ws.random_(0, 256, generator=gen)),
             ("another call's", lambda: run(b)),
             ("zeros", lambda: ws.zero_())]
    for name, fill in fills:
        fill()
        got = run(a)
        torch.cuda.synchronize(dev)
        for t, x, y in zip(("y", "h", "dx", "dA", "dB"), ref, got):
            assert torch.equal(x, y), f"{t} differs on a workspace of {name} bytes"


def test_graph_replays_on_changing_inputs(dev):
    """A captured few-token forward + backward (77 tokens, 5120 x 5120) replayed with other
    activations and output gradients copied into its inputs between replays: every replay
    equals the eager call on those inputs (l and the split partials of one replay are never
    taken for another's)."""
    import torch
    M, K, N, r, c = 77, 5120, 5120, 32, 1.0
    _, d = _case(dev, M, K, N, r, 5300)
    _, e = _case(dev, M, K, N, r, 5400)
    print("[skinny] graph replays on changing inputs", flush=True)
    inputs = [(d["x"], d["dy"]), (e["x"], e["dy"])]
    refs = [_run(dict(d, x=x, dy=dy), c) for x, dy in inputs]
    torch.cuda.synchronize(dev)
    xs, dys = d["x"].clone(), d["dy"].clone()
    stat = dict(d, x=xs, dy=dys)
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        _run(stat, c)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = _run(stat, c)
    torch.cuda.synchronize(dev)
    for rnd in range(6):
        k = rnd % 2
        xs.copy_(inputs[k][0])
        dys.copy_(inputs[k][1])
        g.replay()
        torch.cuda.synchronize(dev)
        for name, a, b in zip(("y", "h", "dx", "dA", "dB"), out, refs[k]):
            assert torch.equal(a, b), f"replay {rnd} (inputs {k}): {name} differs from eager"
