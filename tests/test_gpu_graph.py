"""Every decode op of the path recorded in one HIP graph, in the order of a decode layer pass (the embedding gather,
rmsnorm_q8, gdn_conv_l2 with state snapshots, gated_rmsnorm_q8, sum_norm_q8, swiglu_q8, attn_prep with the q8_0 cache,
quantize_q8_1), replayed several times with eager work and synchronizations in between. Every replay must give the
oracle's bits for every output. The in-place state (the residual x, the conv state planes) is restored before each
replay, so each replay sees the inputs of the first. No op records a memset: the graph holds kernel nodes only."""
import sys

import numpy as np
import pytest

import cfgdata as cd
from conftest import assert_bits_equal

pytestmark = pytest.mark.gpu
E, FF, EPS = cd.E, cd.FF, cd.EPS


def say(msg):
    print(f"[gpu-graph] {msg}", flush=True)
    sys.stdout.flush()


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

        def i32(self, a):
            return self.up(np.asarray(a, np.int32))

    return H()


def test_decode_layer_ops_replay_in_one_graph(q27, oracle, T):
    import torch

    say("decode layer ops in one HIP graph")
    r = cd.rng(4242)
    Tn, C, H, KH = 4, cd.C_CONV, cd.HV, cd.KH
    NQH, NKVH, NCTX, POS = cd.NQH, cd.NKVH, 256, 100
    # inputs
    rows_tab = 64
    table = cd.random_table(r, "iq2_s", rows_tab, E)
    row_bytes = E // 256 * 82
    ids = np.array([5, 63, 0, 5], np.int32)
    x0, part, w = cd.normal(r, Tn * E), cd.normal(r, Tn * E), cd.normal(r, E, 0.1, 1.0)
    cx, cw, st0 = cd.normal(r, Tn * C), cd.normal(r, C * 4, 0.5), cd.normal(r, 4 * C * 3)
    a, b, sa, dtb = cd.normal(r, Tn * H, 2.0), cd.normal(r, Tn * H, 2.0), cd.normal(r, H), cd.normal(r, H)
    o, z, w128 = cd.normal(r, Tn * H * 128), cd.normal(r, Tn * H * 128), cd.normal(r, 128, 0.1, 1.0)
    g, u = cd.normal(r, Tn * FF, 2.0), cd.normal(r, Tn * FF, 2.0)
    qg, k, v = cd.normal(r, Tn * NQH * 512), cd.normal(r, Tn * NKVH * 256), cd.normal(r, Tn * NKVH * 256)
    qw, kw = cd.normal(r, 256, 0.1, 1.0), cd.normal(r, 256, 0.1, 1.0)
    ao = cd.normal(r, Tn * NQH * 256)
    # expected outputs
    e_rows = oracle.get_rows("iq2_s", table, row_bytes, ids, E)
    e_rh, e_rq, e_rd, _ = oracle.rmsnorm_q8(x0, w, E, Tn, EPS)
    e_cy, e_cst, e_cg, e_cb = oracle.gdn_conv_l2(cx, cw, st0, 1, C, Tn, True, 2 * KH, EPS, a, b, sa, dtb, H)
    e_gq, e_gd, e_gs = oracle.gated_rmsnorm_q8(o, w128, z, Tn * H, EPS)
    e_sx, e_sh, e_sq, e_sd = oracle.sum_norm_q8(x0, part, w, E, Tn, EPS)
    e_wq, e_wd, _ = oracle.swiglu_q8(g, u)
    nb = q27.ops.kv_cache_bytes(NKVH, NCTX, True)
    e_kc, e_vc = np.zeros(nb, np.uint8), np.zeros(nb, np.uint8)
    e_qn = oracle.attn_prep(qg, k, v, qw, kw, e_kc, e_vc, POS, Tn, EPS, cd.THETA_SCALE, NQH, NKVH, NCTX, True)
    e_aq, e_ad, _ = oracle.quantize_q8_1(ao, NQH * 256, Tn)
    # device buffers
    d_tab, d_ids, d_rows = T.up(table), T.i32(ids), T.empty(Tn * E)
    d_x, d_xr, d_part, d_w = T.up(x0), T.up(x0), T.up(part), T.up(w)
    d_rh, d_rq, d_rd = T.empty(Tn * E), T.empty(Tn * E, torch.int8), T.empty(Tn * E // 32)
    d_cx, d_cw, d_st, d_pin = T.up(cx), T.up(cw), T.up(st0), T.i32([1])
    d_cy, d_cg, d_cb = T.empty(Tn * C), T.empty(Tn * H), T.empty(Tn * H)
    d_a, d_b, d_sa, d_dtb = T.up(a), T.up(b), T.up(sa), T.up(dtb)
    d_o, d_z, d_w128 = T.up(o), T.up(z), T.up(w128)
    d_gq, d_gd = T.empty(Tn * H * 128, torch.int8), T.empty(Tn * H * 4)
    d_sh, d_sq, d_sd = T.empty(Tn * E), T.empty(Tn * E, torch.int8), T.empty(Tn * E // 32)
    d_g, d_u, d_wq, d_wd = T.up(g), T.up(u), T.empty(Tn * FF, torch.int8), T.empty(Tn * FF // 32)
    d_qg, d_k, d_v, d_qw, d_kw = T.up(qg), T.up(k), T.up(v), T.up(qw), T.up(kw)
    d_qn, d_kc, d_vc, d_pos = T.empty(Tn * NQH * 256), T.empty(nb, torch.uint8), T.empty(nb, torch.uint8), T.i32([POS])
    d_ao, d_aq, d_ad = T.up(ao), T.empty(Tn * NQH * 256, torch.int8), T.empty(Tn * NQH * 8)

    def layer():
        q27.ops.get_rows_iq2_s(d_tab, row_bytes, d_ids, Tn, d_rows, E)
        q27.ops.rmsnorm_q8(d_xr, d_w, d_rh, d_rq, d_rd, E, Tn, EPS)
        q27.ops.gdn_conv_l2(d_cx, d_cw, d_st, d_pin, d_cy, C, Tn, True, 2 * KH, EPS, d_a, d_b, d_sa, d_dtb, d_cg, d_cb, H)
        q27.ops.gated_rmsnorm_q8(d_o, d_w128, d_z, d_gq, d_gd, Tn * H, EPS)
        q27.ops.sum_norm_q8(d_x, d_part, E, Tn, None, d_w, EPS, d_sh, d_sq, d_sd)
        q27.ops.swiglu_q8(d_g, d_u, d_wq, d_wd, Tn * FF)
        q27.ops.attn_prep(d_qg, d_k, d_v, d_qw, d_kw, d_qn, d_kc, d_vc, d_pos, Tn, EPS, cd.THETA_SCALE, NQH, NKVH, NCTX,
                          True, None, None, 0, None, None)
        q27.ops.quantize_q8_1(d_ao, d_aq, d_ad, NQH * 256, Tn)

    def restore():
        d_x.copy_(T.up(x0))
        d_st.copy_(T.up(st0))
        torch.cuda.synchronize()

    def check(tag):
        for got, want, what in ((d_rows, e_rows, "get_rows"), (d_rh, e_rh, "rmsnorm h"), (d_rq, e_rq, "rmsnorm xq"),
                                (d_rd, e_rd, "rmsnorm xd"), (d_cy, e_cy, "conv y"), (d_st, e_cst, "conv planes"),
                                (d_cg, e_cg, "conv g"), (d_cb, e_cb, "conv beta"), (d_gq, e_gq, "gated xq"),
                                (d_gd, e_gd, "gated xd"), (d_x, e_sx, "sum_norm x"), (d_sh, e_sh, "sum_norm h"),
                                (d_sq, e_sq, "sum_norm xq"), (d_sd, e_sd, "sum_norm xd"), (d_wq, e_wq, "swiglu xq"),
                                (d_wd, e_wd, "swiglu xd"), (d_qn, e_qn, "attn qn"), (d_kc, e_kc, "k cache"),
                                (d_vc, e_vc, "v cache"), (d_aq, e_aq, "quantize xq"), (d_ad, e_ad, "quantize xd")):
            assert_bits_equal(T.down(got), want, f"{what} ({tag})")

    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        layer()  # eager, outside the capture
        torch.cuda.synchronize()
        check("eager")
        restore()
        with torch.cuda.graph(graph, stream=s):
            layer()
    for rep in range(4):
        restore()
        graph.replay()
        torch.cuda.synchronize()
        check(f"replay {rep}")
        _ = (d_g * 2).sum().item()  # eager work between replays
