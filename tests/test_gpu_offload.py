"""GPU tests of cpu_offload for int8 frozen weights (reels_amd/offload.py; the reference's
cpu_offload path, src/layers/quantization.jl:46-64, 111-144): codes and scales kept in pinned
host memory, uploaded per call or streamed ahead of use by WeightStreamer. The codes are the same
bytes, so every output must be bit-identical to the resident path."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

bf = torch.bfloat16


def _w(dev, seed, N, K):
    return torch.from_numpy(oracle.normal_bf16(seed, (N, K), 0.02, outlier_rate=1e-3).view(np.int16)
                            ).view(bf).to(dev)


def _same(a, b):
    return torch.equal(a.view(torch.int16) if a.dtype == bf else a,
                       b.view(torch.int16) if b.dtype == bf else b)


def test_move_weight_offload_keeps_pinned_codes(dev):
    from reels_amd import frozen_weight_transfer, move_weight, quantize_frozen_matrix
    w = _w(dev, 1, 384, 256)
    t = frozen_weight_transfer("hip", "bf16", quantization="int8", cpu_offload=True)
    W = move_weight(w, t)
    assert not W.values.is_cuda and W.values.is_pinned() and W.scales.is_pinned()
    ref = quantize_frozen_matrix(w)
    assert torch.equal(W.values, ref.values.cpu())
    assert torch.equal(W.scales.view(torch.int32), ref.scales.cpu().view(torch.int32))
    # re-moving an offloaded weight keeps its pinned codes and scales; moving a resident one
    # offloads it
    again = move_weight(W, t)
    assert again.values is W.values and again.scales is W.scales
    assert not move_weight(ref, t).values.is_cuda


def test_per_call_upload_is_bit_identical(dev):
    from reels_amd import i8lora_backward, i8lora_forward, quantize_frozen_matrix
    from reels_amd.offload import offload_weight
    g = torch.Generator(device=dev).manual_seed(3)
    W = quantize_frozen_matrix(_w(dev, 2, 512, 384))
    Wh = offload_weight(W)
    x = torch.randn((200, 384), generator=g, device=dev).to(bf)
    A = (torch.randn((384, 16), generator=g, device=dev) * 0.01).to(bf)
    B = (torch.randn((16, 512), generator=g, device=dev) * 0.01).to(bf)
    dy = torch.randn((200, 512), generator=g, device=dev).to(bf)
    y1, h1 = i8lora_forward(x, W, A, B, None, 0.5, save_h=True)
    y2, h2 = i8lora_forward(x, Wh, A, B, None, 0.5, save_h=True)
    g1 = i8lora_backward(dy, x, W, A, B, 0.5, h=h1)
    g2 = i8lora_backward(dy, x, Wh, A, B, 0.5, h=h2)
    torch.cuda.synchronize(dev)
    assert _same(y1, y2) and _same(h1, h2)
    for a, b in zip(g1, g2):
        assert _same(a, b)


@pytest.mark.parametrize("slots", [2, 3])
def test_streamed_block_fwd_bwd_is_bit_identical(dev, slots):
    from reels_amd import i8lora_backward, i8lora_forward, quantize_frozen_matrix
    from reels_amd.offload import WeightStreamer, offload_weight, run_streamed
    print(f"[offload] streamed block, {slots} slots", flush=True)
    shapes = [(512, 512), (512, 512), (1536, 512), (512, 1536), (256, 512), (512, 256)]  # (N, K)
    g = torch.Generator(device=dev).manual_seed(11)
    Ws = [quantize_frozen_matrix(_w(dev, 20 + i, N, K)) for i, (N, K) in enumerate(shapes)]
    Hs = [offload_weight(W) for W in Ws]
    M, r = 320, 16
    xs = [torch.randn((M, K), generator=g, device=dev).to(bf) for (N, K) in shapes]
    As = [(torch.randn((K, r), generator=g, device=dev) * 0.01).to(bf) for (N, K) in shapes]
    Bs = [(torch.randn((r, N), generator=g, device=dev) * 0.01).to(bf) for (N, K) in shapes]
    dys = [torch.randn((M, N), generator=g, device=dev).to(bf) for (N, K) in shapes]

    def fwd(i, W):
        return i8lora_forward(xs[i], W, As[i], Bs[i], None, 1.0, save_h=True)

    ref_f = [fwd(i, W) for i, W in enumerate(Ws)]
    ref_b = [i8lora_backward(dys[i], xs[i], Ws[i], As[i], Bs[i], 1.0, h=ref_f[i][1])
             for i in reversed(range(len(Ws)))]
    st = WeightStreamer(dev, slots=slots)
    out_f = run_streamed(Hs, fwd, st)
    order = list(reversed(range(len(Hs))))
    out_b = run_streamed([Hs[i] for i in order],
                         lambda j, W: i8lora_backward(dys[order[j]], xs[order[j]], W, As[order[j]],
                                                      Bs[order[j]], 1.0, h=out_f[order[j]][1]), st)
    torch.cuda.synchronize(dev)
    for (y1, h1), (y2, h2) in zip(ref_f, out_f):
        assert _same(y1, y2) and _same(h1, h2)
    for a, b in zip(ref_b, out_b):
        for t1, t2 in zip(a, b):
            assert _same(t1, t2)
    # one streamed projection (the 512 -> 1536 one) against the oracle: the offloaded codes and
    # scales multiply exactly as the reference's per-call upload would (quantization.jl:46-59)
    from tests._util import assert_parity, bf16_bits, bf16_f32
    i = 2
    q, s = Hs[i].values.numpy(), Hs[i].scales.numpy()
    xb, Ab, Bb, dyb = (bf16_bits(t_) for t_ in (xs[i], As[i], Bs[i], dys[i]))
    yo, ho = oracle.lora_forward(xb, q, s, Ab, Bb, 1.0)
    go = oracle.lora_backward(dyb, xb, q, s, Ab, Bb, 1.0)
    dx, dA, dB = out_b[order.index(i)]
    assert_parity(bf16_f32(out_f[i][0]), yo, "offloaded projection y")
    assert_parity(bf16_f32(out_f[i][1]), ho, "offloaded projection h")
    assert_parity(bf16_f32(dx), go["dx"], "offloaded projection dx")
    assert_parity(dA.cpu().numpy(), go["dA"], "offloaded projection dA")
    assert_parity(dB.cpu().numpy(), go["dB"], "offloaded projection dB")
    # the weights still held when the backward starts are not uploaded again
    assert st.uploads == 2 * len(Hs) - slots


def test_streamer_rejects_when_every_slot_is_held(dev):
    from reels_amd import quantize_frozen_matrix
    from reels_amd.offload import WeightStreamer, offload_weight
    Hs = [offload_weight(quantize_frozen_matrix(_w(dev, 40 + i, 64, 64))) for i in range(3)]
    st = WeightStreamer(dev, slots=2)
    st.acquire(Hs[0])
    st.acquire(Hs[1])
    with pytest.raises(RuntimeError, match="slot"):
        st.prefetch(Hs[2])
    st.release(Hs[0])
    st.prefetch(Hs[2])
    torch.cuda.synchronize(dev)
