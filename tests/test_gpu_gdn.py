"""GPU parity of the Gated-DeltaNet recurrence (q27h_gdn_step through the C ABI, sequential kernel) against the CPU
oracle: bit-exact outputs and state planes for decode (T = 1..4, snapshots on / off, every input plane) and prefill
(flip mode) at the model's head counts (48 value heads on 16 key heads, q / k / v inside one conv-output row), plus the decode ==
prefill identity on the GPU and a graph replay."""
import sys

import numpy as np
import pytest

import cfgdata as cd
from conftest import assert_bits_equal

pytestmark = pytest.mark.gpu

SCALE = np.float32(1.0 / np.sqrt(128.0))


def say(msg):
    print(f"[gpu-gdn] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(autouse=True)
def _sequential_prefill(q27):
    """These tests pin the sequential kernel bit for bit; long prefills otherwise take the chunked form (checked by
    tolerance in test_gpu_gdn_chunked.py)."""
    prev = q27.ops.gdn_prefill_exact(True)
    yield
    q27.ops.gdn_prefill_exact(prev)


def _run(q27, dev, x, stride, g, beta, planes, in_plane, H, HK, T, snapshots, flip):
    import torch

    dx = torch.from_numpy(x).to(dev)
    dp = torch.from_numpy(planes).to(dev)
    pin = torch.tensor([in_plane], dtype=torch.int32, device=dev)
    o = torch.full((max(T, 1) * H * 128,), float("nan"), device=dev)
    q27.ops.gdn_step(dx, dx[HK * 128:], dx[2 * HK * 128:], stride, torch.from_numpy(g).to(dev),
                     torch.from_numpy(beta).to(dev), dp, pin, o, H, HK, T, float(SCALE), snapshots, flip=flip)
    torch.cuda.synchronize()
    return o.cpu().numpy()[: T * H * 128], dp.cpu().numpy()


def _oracle(oracle, x, stride, g, beta, planes, in_plane, H, HK, T, snapshots, flip):
    return oracle.gdn_step(x, x[HK * 128:], x[2 * HK * 128:], stride, g, beta, planes, in_plane, H, HK, T, SCALE,
                           snapshots, flip)


@pytest.mark.parametrize("T", [1, 2, 3, 4])
@pytest.mark.parametrize("snapshots", [True, False])
def test_gdn_decode(q27, oracle, dev, T, snapshots):
    for in_plane in (0, 3):
        say(f"gdn decode T={T} snapshots={snapshots} in_plane={in_plane}")
        x, stride, g, beta, planes = cd.gdn_inputs(cd.rng(100 + 10 * T + in_plane + snapshots), T)
        got_o, got_p = _run(q27, dev, x, stride, g, beta, planes, in_plane, cd.HV, cd.KH, T, snapshots, False)
        want_o, want_p = _oracle(oracle, x, stride, g, beta, planes, in_plane, cd.HV, cd.KH, T, snapshots, False)
        assert_bits_equal(got_o, want_o, f"gdn decode o T={T}")
        assert_bits_equal(got_p, want_p, f"gdn decode planes T={T}")


@pytest.mark.parametrize("M,in_plane", [(2048, 0), (333, 1), (5, 0), (1, 1)])
def test_gdn_prefill(q27, oracle, dev, M, in_plane):
    say(f"gdn prefill M={M} in_plane={in_plane}")
    x, stride, g, beta, planes = cd.gdn_inputs(cd.rng(200 + M), M)
    got_o, got_p = _run(q27, dev, x, stride, g, beta, planes, in_plane, cd.HV, cd.KH, M, False, True)
    want_o, want_p = _oracle(oracle, x, stride, g, beta, planes, in_plane, cd.HV, cd.KH, M, False, True)
    assert_bits_equal(got_o, want_o, f"gdn prefill o M={M}")
    assert_bits_equal(got_p, want_p, f"gdn prefill planes M={M}")


def test_gdn_small_heads_and_edge_values(q27, oracle, dev):
    """One key head per value head (HK = H), H not a multiple of anything, beta 0 / 1, g = 0 and strongly negative."""
    H, HK, M = 5, 5, 70
    say(f"gdn edge H={H} HK={HK} M={M}")
    x, stride, g, beta, planes = cd.gdn_inputs(cd.rng(300), M, H, HK, planes_std=3.0)
    beta[::7] = 0
    beta[1::7] = 1
    g[::5] = 0
    g[2::5] = -60
    got_o, got_p = _run(q27, dev, x, stride, g, beta, planes, 0, H, HK, M, False, True)
    want_o, want_p = _oracle(oracle, x, stride, g, beta, planes, 0, H, HK, M, False, True)
    assert_bits_equal(got_o, want_o, "gdn edge o")
    assert_bits_equal(got_p, want_p, "gdn edge planes")


def test_gdn_prefill_equals_chained_decode_on_gpu(q27, dev):
    import torch

    say("gdn prefill == chained decode")
    M, H, HK = 9, cd.HV, cd.KH
    x, stride, g, beta, planes = cd.gdn_inputs(cd.rng(400), M, H, HK)
    o_pf, p_pf = _run(q27, dev, x, stride, g, beta, planes, 1, H, HK, M, False, True)
    dp = torch.from_numpy(planes).to(dev)
    dp.view(4, -1)[0] = dp.view(4, -1)[1]
    pin = torch.zeros(1, dtype=torch.int32, device=dev)
    dx = torch.from_numpy(x).to(dev).view(M, stride)
    dg, db = torch.from_numpy(g).to(dev).view(M, H), torch.from_numpy(beta).to(dev).view(M, H)
    o = torch.zeros(M, H * 128, device=dev)
    for t in range(M):
        xt = dx[t]
        q27.ops.gdn_step(xt, xt[HK * 128:], xt[2 * HK * 128:], stride, dg[t], db[t], dp, pin, o[t], H, HK, 1,
                         float(SCALE), False)
    torch.cuda.synchronize()
    assert_bits_equal(o.cpu().numpy().reshape(-1), o_pf, "decode chain o")
    assert_bits_equal(dp.cpu().numpy().reshape(4, -1)[0], p_pf.reshape(4, -1)[0], "decode chain state")


def test_gdn_errors(q27, dev):
    import torch

    from qwen27_engine_amd._lib import Q27Error

    H, HK = 2, 1
    stride = 2 * HK * 128 + H * 128
    x = torch.zeros(8 * stride, device=dev)
    g = torch.zeros(8 * H, device=dev)
    planes = torch.zeros(4 * H * 128 * 128, device=dev)
    pin = torch.zeros(1, dtype=torch.int32, device=dev)
    o = torch.zeros(8 * H * 128, device=dev)
    with pytest.raises(Q27Error):  # T > 4 without flip: only 4 snapshot planes
        q27.ops.gdn_step(x, x[128:], x[256:], stride, g, g, planes, pin, o, H, HK, 5, 1.0, True)
    with pytest.raises(Q27Error):  # stride not a multiple of 4 floats
        q27.ops.gdn_step(x, x[128:], x[256:], stride + 1, g, g, planes, pin, o, H, HK, 1, 1.0, True)
    with pytest.raises(Q27Error):  # misaligned k
        q27.ops.gdn_step(x, x[129:], x[256:], stride, g, g, planes, pin, o, H, HK, 1, 1.0, True)


def test_gdn_replays_in_hip_graph(q27, oracle, dev):
    import torch

    say("gdn graph replay")
    H, HK, T = cd.HV, cd.KH, 4
    x, stride, g, beta, planes = cd.gdn_inputs(cd.rng(500), T)
    want_o, want_p = _oracle(oracle, x, stride, g, beta, planes, 2, H, HK, T, True, False)
    dx, dg, db = (torch.from_numpy(a).to(dev) for a in (x, g, beta))
    p0 = torch.from_numpy(planes).to(dev)
    dp = p0.clone()
    pin = torch.full((1,), 2, dtype=torch.int32, device=dev)
    o = torch.zeros(T * H * 128, device=dev)
    s = torch.cuda.Stream()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        q27.ops.gdn_step(dx, dx[HK * 128:], dx[2 * HK * 128:], stride, dg, db, dp, pin, o, H, HK, T, float(SCALE), True)
        torch.cuda.synchronize()
        with torch.cuda.graph(gr, stream=s):
            q27.ops.gdn_step(dx, dx[HK * 128:], dx[2 * HK * 128:], stride, dg, db, dp, pin, o, H, HK, T, float(SCALE),
                             True)
    for _ in range(3):
        dp.copy_(p0)
        o.zero_()
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert_bits_equal(o.cpu().numpy(), want_o, "gdn graph replay o")
        assert_bits_equal(dp.cpu().numpy(), want_p, "gdn graph replay planes")
