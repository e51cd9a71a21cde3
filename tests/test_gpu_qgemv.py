"""GPU parity of the decode GEMV (q27h_qmat_repack + q27h_qgemv through the C ABI) against the CPU oracle:
bit-exact y for every weight type, the model's shapes and 1..4 activation columns."""
import sys

import numpy as np
import pytest

import cfgdata as cd
from conftest import assert_bits_equal

pytestmark = pytest.mark.gpu

TYPES = cd.QG_TYPES


def say(msg):
    print(f"[gpu-qgemv] {msg}", flush=True)
    sys.stdout.flush()


def _run(q27, dev, type_, N, K, raw, xq, xd, ncols):
    import torch

    draw = torch.from_numpy(raw).to(dev)
    m = q27.ops.qmat_upload(draw, type_, N, K)
    y = torch.full((ncols * N,), float("nan"), device=dev)
    q27.ops.qgemv(m, torch.from_numpy(xq).to(dev), torch.from_numpy(xd).to(dev), y, ncols)
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(ncols, N)


@pytest.mark.parametrize("type_", TYPES)
@pytest.mark.parametrize("shape", [(1024, 5120), (6144, 5120), (12288, 5120), (5120, 17408)])
def test_qgemv_model_shapes(q27, oracle, dev, type_, shape):
    N, K = shape
    ncols = 4
    say(f"qgemv type {type_} N={N} K={K} ncols={ncols}")
    r = cd.rng(300 + type_ + N + K)
    raw = cd.random_weights(r, type_, N, K)
    xq, xd = cd.q8_activations(oracle, r, ncols, K)
    got = _run(q27, dev, type_, N, K, raw, xq, xd, ncols)
    want = oracle.qgemv(type_, raw, N, K, xq, xd, ncols)
    assert_bits_equal(got, want, f"qgemv type {type_} {N}x{K}")


@pytest.mark.parametrize("type_", TYPES)
@pytest.mark.parametrize("ncols", [1, 2, 3])
def test_qgemv_columns(q27, oracle, dev, type_, ncols):
    N, K = 2048, 1536  # 6 blocks per row: one wave, slots 6 and 7 idle
    say(f"qgemv type {type_} ncols={ncols}")
    r = cd.rng(400 + type_ + ncols)
    raw = cd.random_weights(r, type_, N, K)
    xq, xd = cd.q8_activations(oracle, r, ncols, K, std=3.0)
    got = _run(q27, dev, type_, N, K, raw, xq, xd, ncols)
    want = oracle.qgemv(type_, raw, N, K, xq, xd, ncols)
    assert_bits_equal(got, want, f"qgemv type {type_} ncols {ncols}")


@pytest.mark.parametrize("type_", TYPES)
@pytest.mark.parametrize("ncols", [1, 2, 3])
def test_qgemv_columns_wide_k(q27, oracle, dev, type_, ncols):
    """One or two columns over long rows: up to 16 waves per tile (K = 17408: 9 waves, 68 blocks in 72 slots;
    K = 32768: 16 waves)."""
    for N, K in [(512, 17408), (64, 32768)]:
        say(f"qgemv type {type_} {N}x{K} ncols={ncols}")
        r = cd.rng(450 + type_ + ncols + K)
        raw = cd.random_weights(r, type_, N, K)
        xq, xd = cd.q8_activations(oracle, r, ncols, K)
        got = _run(q27, dev, type_, N, K, raw, xq, xd, ncols)
        want = oracle.qgemv(type_, raw, N, K, xq, xd, ncols)
        assert_bits_equal(got, want, f"qgemv type {type_} {N}x{K} ncols {ncols}")


def test_qgemv_small_and_edge_shapes(q27, oracle, dev):
    """One tile, one block per row, and partial 8-block groups; zero activations and wide scale ranges."""
    for type_ in TYPES:
        for N, K in [(8, 256), (16, 768), (40, 2304), (16, 40960)]:
            say(f"qgemv edge type {type_} {N}x{K}")
            r = cd.rng(500 + type_ + N)
            raw = cd.random_weights(r, type_, N, K, d_range=(-24, 15))
            xq, xd = cd.q8_activations(oracle, r, 2, K, std=50.0)
            xq[: K // 2] = 0
            got = _run(q27, dev, type_, N, K, raw, xq, xd, 2)
            want = oracle.qgemv(type_, raw, N, K, xq, xd, 2)
            assert_bits_equal(got, want, f"qgemv edge type {type_} {N}x{K}")


def test_qgemv_repack_unaligned_raw(q27, oracle, dev):
    """The repack reads raw rows at any byte alignment: 4-byte loads when every row start allows them, 2-byte loads
    (an odd block count of a 2 mod 4 block size, or a raw pointer at 2 mod 4), byte loads for an odd pointer."""
    import torch

    for type_ in TYPES:
        for N, K, shift in [(24, 1280, 1), (24, 1280, 2), (16, 2304, 3), (8, 256, 1)]:
            say(f"qgemv repack unaligned type {type_} {N}x{K} offset {shift}")
            r = cd.rng(800 + type_ + shift)
            raw = cd.random_weights(r, type_, N, K, d_range=(-20, 10))
            xq, xd = cd.q8_activations(oracle, r, 1, K, std=40.0)
            buf = torch.zeros(raw.size + 16, dtype=torch.uint8, device=dev)
            draw = buf[shift:shift + raw.size]
            draw.copy_(torch.from_numpy(raw))
            assert draw.data_ptr() % 4 == shift % 4
            m = q27.ops.qmat_upload(draw, type_, N, K)
            y = torch.full((N,), float("nan"), device=dev)
            q27.ops.qgemv(m, torch.from_numpy(xq).to(dev), torch.from_numpy(xd).to(dev), y, 1)
            torch.cuda.synchronize()
            want = oracle.qgemv(type_, raw, N, K, xq, xd, 1)
            assert_bits_equal(y.cpu().numpy().reshape(1, N), want, f"repack unaligned {type_} {N}x{K} +{shift}")


def test_qgemv_errors(q27, dev):
    import torch

    from qwen27_engine_amd._lib import Q27Error

    raw = torch.zeros(144 * 8, dtype=torch.uint8, device=dev)
    with pytest.raises(Q27Error):
        q27.ops.qmat_upload(raw, 8, 8, 256)  # Q8_0 is not a GEMV type (neither in the reference)
    m = q27.ops.qmat_upload(raw, cd.Q4_K, 8, 256)
    xq = torch.zeros(5 * 256, dtype=torch.int8, device=dev)
    xd = torch.zeros(5 * 8, device=dev)
    y = torch.zeros(5 * 8, device=dev)
    with pytest.raises(Q27Error):
        q27.ops.qgemv(m, xq, xd, y, 5)
    assert q27.ops.qmat_bytes(cd.Q4_K, 12, 256) == 0  # N % 8


def test_qgemv_replays_in_hip_graph(q27, oracle, dev):
    import torch

    say("qgemv graph replay")
    type_, N, K, ncols = cd.IQ3_S, 1024, 5120, 4
    r = cd.rng(600)
    raw = cd.random_weights(r, type_, N, K)
    xq, xd = cd.q8_activations(oracle, r, ncols, K)
    m = q27.ops.qmat_upload(torch.from_numpy(raw).to(dev), type_, N, K)
    dxq, dxd = torch.from_numpy(xq).to(dev), torch.from_numpy(xd).to(dev)
    y = torch.zeros(ncols * N, device=dev)
    want = oracle.qgemv(type_, raw, N, K, xq, xd, ncols).reshape(-1)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        q27.ops.qgemv(m, dxq, dxd, y, ncols)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            q27.ops.qgemv(m, dxq, dxd, y, ncols)
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert_bits_equal(y.cpu().numpy(), want, "qgemv graph replay")


@pytest.mark.parametrize("type_", [cd.Q6_K, cd.IQ3_S])
def test_qgemv_lm_head_shape(q27, oracle, dev, type_):
    """The output projection (src/model.cu:236): 248320 vocabulary rows x 5120, 31040 tiles in one launch."""
    N, K = 248320, 5120
    say(f"qgemv LM head type {type_} {N}x{K}")
    r = cd.rng(700 + type_)
    raw = cd.random_weights(r, type_, N, K)
    xq, xd = cd.q8_activations(oracle, r, 1, K)
    got = _run(q27, dev, type_, N, K, raw, xq, xd, 1)
    want = oracle.qgemv(type_, raw, N, K, xq, xd, 1)
    assert_bits_equal(got, want, f"qgemv LM head type {type_}")


@pytest.mark.parametrize("type_", TYPES)
@pytest.mark.parametrize("shape,ncols", [((5120, 6144), 4), ((5120, 10240), 4), ((1024, 5120), 3), ((6144, 5120), 2),
                                         ((256, 40960), 1), ((8, 256), 1)])
def test_qgemv_f32_equals_quantize_then_qgemv(q27, oracle, dev, type_, shape, ncols):
    """The fused launch (q8_1 in LDS per workgroup) against quantize_q8_1 followed by qgemv, both through the C ABI,
    and against the CPU oracle: bit-exact y."""
    import torch

    N, K = shape
    say(f"qgemv_f32 type {type_} N={N} K={K} ncols={ncols}")
    r = cd.rng(900 + type_ + N + K + ncols)
    raw = cd.random_weights(r, type_, N, K)
    x = (r.standard_normal(ncols * K) * np.exp(r.standard_normal(ncols * K) * 0.5)).astype(np.float32)
    x[r.choice(x.size, 7, replace=False)] = 0.0
    x[:32] = 0.0  # an all-zero block: q = 0, scale 0
    m = q27.ops.qmat_upload(torch.from_numpy(raw).to(dev), type_, N, K)
    dx = torch.from_numpy(x).to(dev)
    y_f = torch.full((ncols * N,), float("nan"), device=dev)
    q27.ops.qgemv_f32(m, dx, y_f, ncols)
    xq = torch.zeros(ncols * K, dtype=torch.int8, device=dev)
    xd = torch.zeros(ncols * K // 32, device=dev)
    q27.ops.quantize_q8_1(dx, xq, xd, K, ncols)
    y_u = torch.full((ncols * N,), float("nan"), device=dev)
    q27.ops.qgemv(m, xq, xd, y_u, ncols)
    torch.cuda.synchronize()
    assert_bits_equal(y_f.cpu().numpy(), y_u.cpu().numpy(), "y (fused vs quantize + qgemv)")
    oq, od, _ = oracle.quantize_q8_1(x, K, ncols)
    want = oracle.qgemv(type_, raw, N, K, oq, od, ncols)
    assert_bits_equal(y_f.cpu().numpy().reshape(ncols, N), np.asarray(want).reshape(ncols, N), "y (oracle)")
