"""The HIP kernels, through the C ABI, against the committed known answers of tests/golden/known_answers.npz
(inputs and expected outputs from numpy's correctly rounded float32 arithmetic, hand-derived tree sums and exact
closed forms; written by tests/golden/make_golden.py without the oracle). Each case runs at a decode size and,
tiled, at a prefill size, since the two sizes take different kernel variants. Bit-exact."""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "known_answers.npz")
E = 5120
THETA = float(np.float32(1e7) ** np.float32(-2.0 / 64))  # any theta: every angle is 0 in the attn_prep case


def say(msg):
    print(f"[gpu-golden] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def G():
    with np.load(GOLD, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.fixture(scope="module")
def T(dev):
    import torch

    class H:
        def up(self, a):
            return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

        def empty(self, n, dtype=torch.float32):
            return torch.zeros(n, dtype=dtype, device=dev)

        def down(self, t):
            torch.cuda.synchronize()
            return t.cpu().numpy()

    return H()


def same(got, want, what):
    got, want = np.ascontiguousarray(got).ravel(), np.ascontiguousarray(want).ravel()
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    gi = got.view(np.int32) if got.dtype == np.float32 else got
    wi = want.view(np.int32) if want.dtype == np.float32 else want
    bad = np.flatnonzero(gi != wi)
    assert bad.size == 0, f"{what}: {bad.size} of {got.size} differ, first {bad[0]}: {got[bad[0]]!r} vs {want[bad[0]]!r}"


@pytest.mark.parametrize("reps", [1, 64])
def test_quantize_q8_1_golden_on_gpu(q27, T, G, reps):
    import torch

    say(f"quantize_q8_1 golden reps={reps}")
    x = np.tile(G["q8_x"], reps)
    n = x.size
    xq, xd, xs = T.empty(n, torch.int8), T.empty(n // 32), T.empty(n // 16)
    q27.ops.quantize_q8_1(T.up(x), xq, xd, 256, n // 256, None, xs)
    same(T.down(xq), np.tile(G["q8_xq"], reps), "xq")
    same(T.down(xd), np.tile(G["q8_xd"], reps), "xd")
    same(T.down(xs), np.tile(G["q8_xs"], reps), "xs")


@pytest.mark.parametrize("i", range(4))
@pytest.mark.parametrize("rows", [1, 258])
def test_rmsnorm_q8_golden_on_gpu(q27, T, G, i, rows):
    import torch

    say(f"rmsnorm_q8 golden row {i} rows={rows}")
    x = np.tile(G[f"row{i}_x"], rows)
    h, xq, xd, xs = T.empty(rows * E), T.empty(rows * E, torch.int8), T.empty(rows * E // 32), T.empty(rows * E // 16)
    q27.ops.rmsnorm_q8(T.up(x), T.up(G[f"row{i}_w"]), h, xq, xd, E, rows, float(G[f"row{i}_eps"]), None, xs)
    same(T.down(h), np.tile(G[f"row{i}_h"], rows), f"row {i} h")
    same(T.down(xq), np.tile(G[f"row{i}_xq"], rows), f"row {i} xq")
    same(T.down(xd), np.tile(G[f"row{i}_xd"], rows), f"row {i} xd")
    same(T.down(xs), np.tile(G[f"row{i}_xs"], rows), f"row {i} xs")


@pytest.mark.parametrize("i", range(2))
@pytest.mark.parametrize("heads", [1, 4096])
def test_l2norm_golden_on_gpu(q27, T, G, i, heads):
    say(f"l2norm_heads golden head {i} heads={heads}")
    xd = T.up(np.tile(G[f"l2{i}_x"], heads))
    q27.ops.l2norm_heads(xd, 128, heads, 1, 128 * heads, float(G[f"l2{i}_eps"]))
    same(T.down(xd), np.tile(G[f"l2{i}_y"], heads), f"l2 head {i}")


@pytest.mark.parametrize("reps", [1, 256])
def test_get_rows_q8_0_golden_on_gpu(q27, T, G, reps):
    say(f"get_rows_q8_0 golden reps={reps}")
    ids = np.tile(G["q80_ids"], reps)
    y = T.empty(ids.size * E)
    q27.ops.get_rows_q8_0(T.up(G["q80_table"]), 34 * (E // 32), T.up(ids.astype(np.int32)), ids.size, y, E)
    same(T.down(y), np.tile(G["q80_y"], reps), "q8_0 rows")


@pytest.mark.parametrize("reps", [1, 128])
def test_attn_prep_golden_on_gpu(q27, T, G, reps):
    """reps = 1: the 4-token decode form; reps = 128: the 4 tokens repeated to 512 (one workgroup per token), the
    cache rows of token t being those of token t % 4 at row pos0 + t."""
    import torch

    say(f"attn_prep golden reps={reps}")
    nqh, nkvh, pos0, nctx0 = 24, 4, int(G["att_pos0"]), int(G["att_nctx"])
    Tn = 4 * reps
    nctx = nctx0 if reps == 1 else 1024
    nb = nkvh * nctx * 272
    kc, vc = T.empty(nb, torch.uint8), T.empty(nb, torch.uint8)
    qn = T.empty(Tn * nqh * 256)
    q27.ops.attn_prep(T.up(np.tile(G["att_qg"], reps)), T.up(np.tile(G["att_k"], reps)), T.up(np.tile(G["att_v"], reps)),
                      T.up(G["att_qw"]), T.up(G["att_kw"]), qn, kc, vc, T.up(np.array([pos0], np.int32)), Tn,
                      float(G["att_eps"]), THETA, nqh, nkvh, nctx, True, None, None, 0,
                      T.up(np.zeros((Tn, 3), np.int32)), None)
    same(T.down(qn), np.tile(G["att_qn"], reps), "qn")
    so0, so = nkvh * nctx0 * 256, nkvh * nctx * 256
    for got, gold, what in ((kc, G["att_kc"], "k cache"), (vc, G["att_vc"], "v cache")):
        want = np.zeros(nb, np.uint8)
        for h in range(nkvh):
            for t in range(Tn):
                r0, r = h * nctx0 + pos0 + t % 4, h * nctx + pos0 + t
                want[r * 256:(r + 1) * 256] = gold[r0 * 256:(r0 + 1) * 256]
                want[so + r * 16:so + (r + 1) * 16] = gold[so0 + r0 * 16:so0 + (r0 + 1) * 16]
        same(T.down(got), want, what)
