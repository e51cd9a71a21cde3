"""Benchmark of the fused per-layer ops on one MI355X.

Metric: achieved HBM GB/s (and % of 8 TB/s) per fused op; us per decode step; us per 2048-token
prefill batch. A "step" is one 2048-token prefill pass over the in-scope launches of the 64 layers,
in the order of Decoder::prefill_batch / pf_layer (src/model.cu:1201-1243, 1280-1294):

  get_rows_iq2_s, rmsnorm_q8 (h, xs), then per layer
    GDN layer (48):  gdn_conv_prefill, gated_rmsnorm_q8 (xs), sum_norm_rows, swiglu_q8 (xs), sum_norm_rows
    attn layer (16): attn_prep (q8_0 cache), quantize_q8_1 (xs), sum_norm_rows, swiglu_q8 (xs), sum_norm_rows

`value` = algorithmic bytes of the step / its time (inputs resident in HBM). Beside it: the decode verify pass
(configs[1], T = 4: the 306 in-scope launches recorded in one HIP graph, median replay time), per-op GB/s from
per-launch HIP events inside the prefill pass, the roofline of the dominant kernel (swiglu_q8), and the CPU oracle
timed on a bounded sample of the same pass. Synthetic data, random weights of the model's shapes.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "qwen27-engine_amd")

E, FF, NQH, NKVH, KH, HV, D = 5120, 17408, 24, 4, 16, 48, 128
C = 2 * KH * D + HV * D
N_LAYER, N_CTX, VOCAB = 64, 180224, 248320
EPS = 1e-6
HBM_PEAK_GBS = 8000.0
# HBM bytes per swiglu_q8 launch at M = 2048, measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE over the prefill
# pass and scaled by the copy-kernel calibration (FETCH x 2.000, WRITE x 1.000): 139291 KiB and 47872 KiB
# (profiles/hbm_traffic_prefill_pass.md). The counters cannot be read from inside this process.
SWIGLU_TRAFFIC_BYTES = int((139291 * 2.0 + 47872 * 1.0) * 1024)


def is_attn(il):
    return (il + 1) % 4 == 0  # src/model.h:27


# ---------------------------------------------------------------- algorithmic bytes per unit of each op (read + write, compulsory)
def bytes_rmsnorm_q8(rows, h, xs):
    return rows * (20480 + (20480 if h else 0) + 5120 + 640 + (1280 if xs else 0)) + 20480


def bytes_sum_norm(rows, h, xs):
    return rows * (3 * 20480 + (20480 if h else 0) + 5120 + 640 + (1280 if xs else 0)) + 20480


def bytes_swiglu_q8(n, xs):
    return int(n * (8 + 1 + 0.125 + (0.25 if xs else 0)))


def bytes_quantize(n, xs):
    return int(n * (4 + 1 + 0.125 + (0.25 if xs else 0)))


def bytes_gated(heads, xs):
    return heads * (512 + 512 + 128 + 16 + (32 if xs else 0)) + 512


def bytes_attn_prep(T):
    return T * (NQH * 256 * 4 * 2 + NKVH * 256 * 4 * 2 + 2 * NKVH * (256 + 16)) + 2 * 1024


def bytes_gdn_conv(T):
    return T * (2 * C * 4 + 4 * HV * 4) + C * 16 + 2 * C * 12 + HV * 8


def bytes_get_rows(T, uniq, row_bytes):
    return T * E * 4 + uniq * row_bytes + T * 4


# ---------------------------------------------------------------- helpers
def load_package():
    name = "qwen27_engine_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Pass:
    """Buffers and launch list of one pass (prefill M rows, or the decode verify pass at T rows)."""

    def __init__(self, q27, torch, M, decode, seed=7, cold=False):
        """cold: every layer reads inputs of its own (the partial sums, gate/up, conv input, o/z, q/k/v, attention
        output) and the residual rotates over 8 buffers, so no launch finds its inputs in the 256 MB MALL, as in
        the engine where each layer's GEMMs stream far more than 256 MB between two uses of a buffer."""
        self.q27, self.torch, self.M, self.decode, self.cold = q27, torch, M, decode, cold
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev)
        g.manual_seed(seed)

        def randn(n, std=1.0, mean=0.0):
            return torch.randn(n, device=dev, generator=g) * std + mean

        def zeros(n, dtype=torch.float32):
            return torch.zeros(n, dtype=dtype, device=dev)

        f = torch.float32
        nl = N_LAYER if cold else 1
        self.scale = torch.exp(randn(E))
        self.xs_ring = [(randn(M * E).view(M, E) * self.scale).to(torch.bfloat16).to(f).reshape(-1)
                        for _ in range(8 if cold else 1)]
        self.x = self.xs_ring[0]
        self.x0s = [x.clone() for x in self.xs_ring]
        self.m_outs = [randn(M * E) for _ in range(2 * nl)]
        self.h = zeros(M * E)
        self.xq = zeros(M * FF, torch.int8)
        self.xd = zeros(M * FF // 32)
        self.xs = zeros(M * FF // 16)
        self.norm_w = [randn(E, 0.1, 1.0) for _ in range(2 * N_LAYER + 1)]
        # GDN
        nlg, nla = (48, 16) if cold else (1, 1)
        self.qkvs = [randn(M * C) for _ in range(nlg)]
        self.conv = zeros(M * C)
        self.conv_w = [randn(C * 4, 0.5) for _ in range(48)]
        self.planes = [randn(4 * C * 3) for _ in range(48)]
        self.dplane = torch.zeros(1, dtype=torch.int32, device=dev)
        self.ab = randn(2 * M * HV, 2.0)
        self.ssm_a, self.dt_bias = randn(HV), randn(HV)
        self.gg, self.beta = zeros(M * HV), zeros(M * HV)
        self.ozs = [(randn(M * HV * D), randn(M * HV * D)) for _ in range(nlg)]
        self.ssm_norm = randn(D, 0.1, 1.0)
        # FFN
        self.fgus = [(randn(M * FF, 2.0), randn(M * FF, 2.0)) for _ in range(nl)]
        self.fg, self.fu = self.fgus[0]
        # attention
        self.qkvas = [(randn(M * NQH * 512), randn(M * NKVH * 256), randn(M * NKVH * 256)) for _ in range(nla)]
        self.q_norm, self.k_norm = randn(256, 0.1, 1.0), randn(256, 0.1, 1.0)
        self.qn = zeros(M * NQH * 256)
        self.attn_os = [randn(M * NQH * 256) for _ in range(nla)]
        cache_bytes = q27.ops.kv_cache_bytes(NKVH, N_CTX, True)
        self.kc = [zeros(cache_bytes, torch.uint8) for _ in range(16)]
        self.vc = [zeros(cache_bytes, torch.uint8) for _ in range(16)]
        self.pos0 = torch.tensor([150000 if decode else 131072], dtype=torch.int32, device=dev)
        self.rdelta = torch.zeros(1, dtype=torch.int32, device=dev)
        self.theta_scale = float(torch.tensor(1e7, dtype=f) ** torch.tensor(-2.0 / 64, dtype=f))
        # token embedding: IQ2_S table (the reference's embedding type), random blocks with finite fp16 scales
        self.row_bytes = E // 256 * 82
        tab = torch.randint(0, 256, (VOCAB * (E // 256), 82), dtype=torch.uint8, device=dev, generator=g)
        dsc = (torch.exp2(torch.rand(VOCAB * (E // 256), device=dev, generator=g) * 6 - 10)).to(torch.float16)
        tab[:, 0:2] = dsc.view(torch.uint8).view(-1, 2)
        self.table = tab.reshape(-1)
        ids = self._zipf_ids(M, g, dev)
        self.ids = ids
        self.uniq = int(torch.unique(ids).numel())
        self.launches = self._build()

    def _zipf_ids(self, M, g, dev):
        torch = self.torch
        w = torch.arange(1, VOCAB + 1, dtype=torch.float64, device=dev) ** -1.1
        cdf = torch.cumsum(w, 0)
        cdf /= cdf[-1].clone()
        u = torch.rand(M, dtype=torch.float64, device=dev, generator=g)
        ranks = torch.clamp(torch.searchsorted(cdf, u), max=VOCAB - 1)
        perm = torch.randperm(VOCAB, device=dev, generator=g)
        return perm[ranks].to(torch.int32)

    def _build(self):
        """[(op name, algorithmic bytes, callable)] in launch order."""
        o, M, dec = self.q27.ops, self.M, self.decode
        L = []
        x0 = self.xs_ring[0]
        L.append(("get_rows_iq2_s", bytes_get_rows(M, self.uniq, self.row_bytes),
                  lambda: o.get_rows_iq2_s(self.table, self.row_bytes, self.ids, M, x0, E)))
        xs0 = None if dec else self.xs
        L.append(("rmsnorm_q8", bytes_rmsnorm_q8(M, True, not dec),
                  lambda: o.rmsnorm_q8(x0, self.norm_w[0], self.h, self.xq, self.xd, E, M, EPS, None, xs0)))
        ig = ia = 0
        pick = lambda seq, i: seq[i % len(seq)]  # noqa: E731
        for il in range(N_LAYER):
            x = pick(self.xs_ring, il)
            if not is_attn(il):
                qkv, (oo, zz) = pick(self.qkvs, ig), pick(self.ozs, ig)
                gi = ig
                ab2 = self.ab[M * HV:]
                if dec:
                    L.append(("gdn_conv_l2", bytes_gdn_conv(M),
                              lambda gi=gi, ab2=ab2, qkv=qkv: o.gdn_conv_l2(qkv, self.conv_w[gi], self.planes[gi], self.dplane,
                                                                            self.conv, C, M, True, 2 * KH, EPS, self.ab, ab2,
                                                                            self.ssm_a, self.dt_bias, self.gg, self.beta, HV)))
                else:
                    L.append(("gdn_conv_prefill", bytes_gdn_conv(M),
                              lambda gi=gi, ab2=ab2, qkv=qkv: o.gdn_conv_prefill(qkv, self.conv_w[gi], self.planes[gi],
                                                                                 self.dplane, self.conv, C, M, 2 * KH, EPS,
                                                                                 self.ab, ab2, self.ssm_a, self.dt_bias,
                                                                                 self.gg, self.beta, HV)))
                L.append(("gated_rmsnorm_q8", bytes_gated(M * HV, not dec),
                          lambda oo=oo, zz=zz: o.gated_rmsnorm_q8(oo, self.ssm_norm, zz, self.xq, self.xd, M * HV, EPS, None,
                                                                  None if dec else self.xs)))
                ig += 1
            else:
                ai = ia
                (qg, kk, vv), ao = pick(self.qkvas, ia), pick(self.attn_os, ia)
                L.append(("attn_prep", bytes_attn_prep(M),
                          lambda ai=ai, qg=qg, kk=kk, vv=vv: o.attn_prep(qg, kk, vv, self.q_norm, self.k_norm, self.qn,
                                                                         self.kc[ai], self.vc[ai], self.pos0, M, EPS,
                                                                         self.theta_scale, NQH, NKVH, N_CTX, True, None, None,
                                                                         0, None, self.rdelta)))
                if not dec:  # decode fuses this quantization into attention (src/model.cu:727-731)
                    L.append(("quantize_q8_1", bytes_quantize(M * NQH * 256, True),
                              lambda ao=ao: o.quantize_q8_1(ao, self.xq, self.xd, NQH * 256, M, None, self.xs)))
                ia += 1
            w1, w2 = self.norm_w[2 * il + 1], self.norm_w[2 * il + 2]
            p1, p2 = pick(self.m_outs, 2 * il), pick(self.m_outs, 2 * il + 1)
            fg, fu = pick(self.fgus, il)
            nxt_gdn = il + 1 < N_LAYER and not is_attn(il + 1)
            h2 = self.h if nxt_gdn else None
            if dec:
                L.append(("sum_norm_q8", bytes_sum_norm(M, False, False),
                          lambda w1=w1, x=x, p1=p1: o.sum_norm_q8(x, p1, E, M, None, w1, EPS, None, self.xq, self.xd)))
            else:
                L.append(("sum_norm_rows", bytes_sum_norm(M, False, True),
                          lambda w1=w1, x=x, p1=p1: o.sum_norm_rows(x, p1, E, M, None, w1, EPS, None, self.xq, self.xd,
                                                                    self.xs)))
            L.append(("swiglu_q8", bytes_swiglu_q8(M * FF, not dec),
                      lambda fg=fg, fu=fu: o.swiglu_q8(fg, fu, self.xq, self.xd, M * FF, None, None if dec else self.xs)))
            if dec:
                L.append(("sum_norm_q8", bytes_sum_norm(M, h2 is not None, False),
                          lambda w2=w2, h2=h2, x=x, p2=p2: o.sum_norm_q8(x, p2, E, M, None, w2, EPS, h2, self.xq, self.xd)))
            else:
                L.append(("sum_norm_rows", bytes_sum_norm(M, h2 is not None, True),
                          lambda w2=w2, h2=h2, x=x, p2=p2: o.sum_norm_rows(x, p2, E, M, None, w2, EPS, h2, self.xq, self.xd,
                                                                           self.xs)))
        return L

    def reset(self):
        for x, x0 in zip(self.xs_ring, self.x0s):
            x.copy_(x0)

    def bytes_per_step(self):
        return sum(b for _, b, _ in self.launches)

    def run(self):
        for _, _, fn in self.launches:
            fn()

    def run_events(self, acc):
        """One pass with a HIP event pair around every launch; accumulates (op -> [sum_ms, count, bytes])."""
        torch = self.torch
        evs = []
        for name, b, fn in self.launches:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            evs.append((name, b, e0, e1))
        torch.cuda.synchronize()
        for name, b, e0, e1 in evs:
            a = acc.setdefault(name, [0.0, 0, 0])
            a[0] += e0.elapsed_time(e1)
            a[1] += 1
            a[2] += b


def _cpu_shared(seed=5):
    """Inputs the CPU threads share, at the GPU pass's shapes: the 248320 x 5120 IQ2_S table (407 MB, random blocks,
    fp16 scales in [2^-10, 2^-4]) and one layer's q8_0 K / V cache of 180224 rows (each thread writes its own rows)."""
    import numpy as np

    sys.path.insert(0, ROOT)
    from oracle import q27_oracle as O

    r = np.random.default_rng(seed)
    table = r.bit_generator.random_raw(VOCAB * 1640 // 8).view(np.uint8)
    d = np.exp2(r.random(VOCAB * 20) * 6 - 10).astype(np.float16)
    table.reshape(-1, 82)[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    w = np.arange(1, VOCAB + 1, dtype=np.float64) ** -1.1
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    kc = np.zeros(O.kv_cache_bytes(NKVH, N_CTX, True), np.uint8)
    return {"table": table, "cdf": cdf, "perm": r.permutation(VOCAB), "kc": kc, "vc": np.zeros_like(kc)}


def _cpu_pass(M, seed, sh, pos0, per_op=None):
    """The CPU oracle (scalar C) over the 322 launches of one prefill pass restricted to M token rows at the GPU
    pass's shapes (Zipf ids into the full IQ2_S table, cache rows pos0 .. pos0 + M - 1 of a 180224-row q8_0 cache).
    Returns the algorithmic bytes it moved (the same per-row definitions as the GPU step). per_op, if given,
    accumulates op -> [seconds, bytes]."""
    import numpy as np

    sys.path.insert(0, ROOT)
    from oracle import q27_oracle as O

    r = np.random.default_rng(seed)
    f = lambda n, s=1.0, m=0.0: (r.standard_normal(n) * s + m).astype(np.float32)  # noqa: E731
    x, part, w = f(M * E), f(M * E), f(E, 0.1, 1.0)
    g, u = f(M * FF, 2.0), f(M * FF, 2.0)
    o, z, w128 = f(M * HV * D), f(M * HV * D), f(D, 0.1, 1.0)
    qkv, cw, planes = f(M * C), f(C * 4, 0.5), f(4 * C * 3)
    ab, sa, dtb = f(2 * M * HV, 2.0), f(HV), f(HV)
    qg, k, v, qw, kw = f(M * NQH * 512), f(M * NKVH * 256), f(M * NKVH * 256), f(256, 0.1, 1.0), f(256, 0.1, 1.0)
    attn_o = f(M * NQH * 256)
    ids = sh["perm"][np.minimum(np.searchsorted(sh["cdf"], r.random(M)), VOCAB - 1)].astype(np.int32)
    ts = float(np.float32(1e7) ** np.float32(-2.0 / 64))
    total = 0

    def run(name, nbytes, fn):
        nonlocal total
        t0 = time.perf_counter()
        fn()
        if per_op is not None:
            acc = per_op.setdefault(name, [0.0, 0])
            acc[0] += time.perf_counter() - t0
            acc[1] += nbytes
        total += nbytes

    run("get_rows_iq2_s", bytes_get_rows(M, len(np.unique(ids)), 1640), lambda: O.get_rows("iq2_s", sh["table"], 1640, ids, E))
    run("rmsnorm_q8", bytes_rmsnorm_q8(M, True, True), lambda: O.rmsnorm_q8(x, w, E, M, EPS, with_h=True, with_xs=True))
    for il in range(N_LAYER):
        if not is_attn(il):
            run("gdn_conv_prefill", bytes_gdn_conv(M),
                lambda: O.gdn_conv_prefill(qkv, cw, planes, 0, C, M, 2 * KH, EPS, ab[:M * HV], ab[M * HV:], sa, dtb, HV))
            run("gated_rmsnorm_q8", bytes_gated(M * HV, True), lambda: O.gated_rmsnorm_q8(o, w128, z, M * HV, EPS, with_xs=True))
        else:
            run("attn_prep", bytes_attn_prep(M),
                lambda: O.attn_prep(qg, k, v, qw, kw, sh["kc"], sh["vc"], pos0, M, EPS, ts, NQH, NKVH, N_CTX, True))
            run("quantize_q8_1", bytes_quantize(M * NQH * 256, True), lambda: O.quantize_q8_1(attn_o, NQH * 256, M, with_xs=True))
        run("sum_norm_rows", bytes_sum_norm(M, False, True), lambda: O.sum_norm_rows(x, part, w, E, M, EPS))
        run("swiglu_q8", bytes_swiglu_q8(M * FF, True), lambda: O.swiglu_q8(g, u, with_xs=True))
        run("sum_norm_rows", bytes_sum_norm(M, False, True), lambda: O.sum_norm_rows(x, part, w, E, M, EPS))
    return total


def cpu_baseline(rows, threads, sh, per_op=None):
    """The oracle on a bounded sample of the prefill pass: `rows` token rows split over `threads` host threads (the
    C calls release the GIL), each thread on its own rows and cache positions. Returns (GB/s, seconds)."""
    from concurrent.futures import ThreadPoolExecutor

    per = max(1, rows // threads)
    t0 = time.perf_counter()
    if threads == 1:
        total = _cpu_pass(per, 5, sh, 131072, per_op)
    else:
        with ThreadPoolExecutor(threads) as ex:
            total = sum(ex.map(lambda i: _cpu_pass(per, 5 + i, sh, 131072 + i * per), range(threads)))
    dt = time.perf_counter() - t0
    return total / dt / 1e9, dt


def host_cpu_info():
    """Host core counts and model name (lscpu), recorded beside the CPU baseline."""
    import subprocess

    info = {"os_cpu_count": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0))}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core"):
                info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return info


def time_back_to_back(torch, fn, reps):
    """Average launch time of `fn(i)` over `reps` back-to-back launches between two HIP events (3 warm-up launches)."""
    for i in range(3):
        fn(i)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(reps):
        fn(i)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / reps


def time_graph(torch, fn, n):
    """Median time per launch of `fn` when n launches are replayed from one HIP graph (decode-sized ops)."""
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            for _ in range(n):
                fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(20):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b) * 1e3 / n)
    ts.sort()
    return ts[len(ts) // 2]


def bench_gathers(q27, torch, T=2048, U=4):
    """248320 x 5120 tables, 2048 Zipf(1.1) ids + 4 uniform ids -> f32 rows. GB/s on compulsory bytes
    (rows written + distinct table rows read) and on logical bytes (every id's table row counted)."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    w = torch.arange(1, VOCAB + 1, dtype=torch.float64, device=dev) ** -1.1
    cdf = torch.cumsum(w, 0)
    cdf /= cdf[-1].clone()
    ranks = torch.clamp(torch.searchsorted(cdf, torch.rand(T, dtype=torch.float64, device=dev, generator=g)), max=VOCAB - 1)
    perm = torch.randperm(VOCAB, device=dev, generator=g)
    ids = torch.cat([perm[ranks], torch.randint(0, VOCAB, (U,), device=dev, generator=g)]).to(torch.int32)
    nid = ids.numel()
    uniq = int(torch.unique(ids).numel())
    y = torch.empty(nid * E, device=dev)
    out = {}
    for kind, bb, bv, doffs in (("q4_k", 144, 256, (0, 2)), ("q6_k", 210, 256, (208,)), ("q8_0", 34, 32, (0,)),
                                ("iq2_s", 82, 256, (0,))):
        nblk = VOCAB * (E // bv)
        tab = torch.randint(0, 256, (nblk, bb), dtype=torch.uint8, device=dev, generator=g)
        for off in doffs:
            d = torch.exp2(torch.rand(nblk, device=dev, generator=g) * 6 - 10).to(torch.float16)
            tab[:, off:off + 2] = d.view(torch.uint8).view(-1, 2)
        row_bytes = E // bv * bb
        fn = getattr(q27.ops, "get_rows_" + kind)
        us = time_back_to_back(torch, lambda i: fn(tab, row_bytes, ids, nid, y, E), 20)
        comp = nid * E * 4 + uniq * row_bytes
        logical = nid * (E * 4 + row_bytes)
        out[kind] = {"us": round(us, 2), "GBps_compulsory": round(comp / us / 1e3, 1),
                     "GBps_logical": round(logical / us / 1e3, 1), "distinct_ids": uniq, "ids": nid}
        log(f"  gather {kind:6s} {us:7.2f} us  {comp / us / 1e3:7.1f} GB/s compulsory  {logical / us / 1e3:7.1f} GB/s logical")
        del tab
    return out


def bench_multimodal(q27, torch, M=4099):
    """4099 rows (3 text + a 64 x 64 image grid): gated_rmsnorm_q8 over 48 value heads, l2norm_heads of
    the 32 q/k heads (row stride 10240, in place), attn_prep with IMRoPE positions (t, h, w)."""
    dev = torch.device("cuda:0")
    rn = lambda n: torch.randn(n, device=dev)  # noqa: E731
    sets = 3
    o = [rn(M * HV * D) for _ in range(sets)]
    z = [rn(M * HV * D) for _ in range(sets)]
    w128 = rn(D) * 0.1 + 1
    xq = torch.empty(M * HV * D, dtype=torch.int8, device=dev)
    xd = torch.empty(M * HV * D // 32, device=dev)
    xs = torch.empty(M * HV * D // 16, device=dev)
    res = {}
    us = time_back_to_back(torch, lambda i: q27.ops.gated_rmsnorm_q8(o[i % sets], w128, z[i % sets], xq, xd, M * HV, EPS, None, xs), 21)
    b = bytes_gated(M * HV, True)
    res["gated_rmsnorm_q8"] = {"us": round(us, 2), "GBps": round(b / us / 1e3, 1), "bytes": b}
    del o, z
    conv = [rn(M * C) for _ in range(sets)]
    us = time_back_to_back(torch, lambda i: q27.ops.l2norm_heads(conv[i % sets], D, 2 * KH, M, C, EPS), 21)
    b = M * 2 * KH * D * 8
    res["l2norm_heads"] = {"us": round(us, 2), "GBps": round(b / us / 1e3, 1), "bytes": b}
    del conv
    rows = [(p, p, p) for p in range(3)] + [(3, 3 + i // 64, 3 + i % 64) for i in range(4096)]
    rope3 = torch.tensor(rows, dtype=torch.int32, device=dev).reshape(-1)
    qg = [rn(M * NQH * 512) for _ in range(sets)]
    k, v = rn(M * NKVH * 256), rn(M * NKVH * 256)
    qn = torch.empty(M * NQH * 256, device=dev)
    n_ctx = 8192
    cb = q27.ops.kv_cache_bytes(NKVH, n_ctx, True)
    kc, vc = torch.zeros(cb, dtype=torch.uint8, device=dev), torch.zeros(cb, dtype=torch.uint8, device=dev)
    pos0 = torch.zeros(1, dtype=torch.int32, device=dev)
    ts = float(torch.tensor(1e7) ** torch.tensor(-2.0 / 64))
    us = time_back_to_back(torch, lambda i: q27.ops.attn_prep(qg[i % sets], k, v, w128.repeat(2), w128.repeat(2), qn, kc, vc,
                                                                pos0, M, EPS, ts, NQH, NKVH, n_ctx, True, None, None, 0,
                                                                rope3, None), 21)
    b = bytes_attn_prep(M)
    res["attn_prep_imrope"] = {"us": round(us, 2), "GBps": round(b / us / 1e3, 1), "bytes": b}
    for k_, v_ in res.items():
        log(f"  cfg5 {k_:18s} {v_['us']:7.2f} us  {v_['GBps']:7.1f} GB/s")
    return res


GEMV_TYPES = {"iq3_s": (21, 110, (0,)), "q4_k": (12, 144, (0, 2)), "q6_k": (14, 210, (208,)), "iq4_xs": (23, 136, (0,)),
              "q2_k": (10, 84, (80, 82)), "iq2_xxs": (16, 66, (0,)), "iq2_xs": (17, 74, (0,)), "iq3_xxs": (18, 98, (0,)),
              "iq2_s": (22, 82, (0,)), "iq1_m": (29, 56, ())}
# decode GEMV shapes of the model (N outputs x K inputs, tp = 1): wk / wv, ssm_out / wo, gate z, qkv, wq,
# ffn up / gate, ffn down (src/model.cu:715-796)
GEMV_SHAPES = [(1024, 5120), (5120, 6144), (6144, 5120), (10240, 5120), (12288, 5120), (17408, 5120), (5120, 17408)]


def gemv_profile(type_, N, K, T):
    """Eight qgemv launches of one shape over four uploaded copies of a random matrix (for counter runs)."""
    import torch

    q27 = load_package()
    q27.lib()
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(21)
    bb = {10: 84, 12: 144, 14: 210, 16: 66, 17: 74, 18: 98, 21: 110, 22: 82, 23: 136, 29: 56}[type_]
    raw = torch.randint(0, 256, (N * (K // 256) * bb,), dtype=torch.uint8, device=dev, generator=g)
    mats = [q27.ops.qmat_upload(raw, type_, N, K) for _ in range(4)]
    xq = torch.randint(-127, 128, (T * K,), dtype=torch.int8, device=dev, generator=g)
    xd = torch.rand(T * K // 32, device=dev, generator=g) * 0.01
    y = torch.empty(T * N, device=dev)
    for i in range(8):
        q27.ops.qgemv(mats[i % 4], xq, xd, y, T)
    torch.cuda.synchronize()
    log(f"gemv profile: type {type_} {N}x{K} T={T}, 8 launches")


def bench_gemv(q27, torch):
    """Decode GEMV (the consumer of the q8_1 activations, src/qgemv.cu): per weight type and model shape, us per
    launch and GB/s of (matrix bytes + activations + y) with T = 4 and T = 1 activation columns. Enough distinct
    matrices are cycled that no launch finds its weights in the 256 MB MALL (as in a decode step, which streams
    all 64 layers' weights); the launches are replayed from one HIP graph whose nodes walk the matrices, as a decode
    step's graph issues them (launched one by one from Python, launches of up to about 10 us measured the host's
    launch rate; in the graph each figure includes the node's own cost, about 1.5 us)."""
    import math

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(13)
    out = {}
    for name, (tid, bb, doffs) in GEMV_TYPES.items():
        res = {}
        for N, K in (GEMV_SHAPES if name == "iq3_s" else [(17408, 5120), (5120, 17408)]):
            nbytes = q27.ops.qmat_bytes(tid, N, K)
            cnt = max(3, math.ceil(600e6 / nbytes))
            raw = torch.randint(0, 256, (N * (K // 256), bb), dtype=torch.uint8, device=dev, generator=g)
            for off in doffs:
                d = torch.exp2(torch.rand(raw.shape[0], device=dev, generator=g) * 6 - 10).to(torch.float16)
                raw[:, off:off + 2] = d.view(torch.uint8).view(-1, 2)
            if name == "iq1_m":  # the fp16 scale is the four top nibbles of the scales words: keep it finite
                raw[:, 49:56:2] &= 0x0F
                raw[:, 55] |= 0x20
            mats = [q27.ops.qmat_upload(raw.reshape(-1), tid, N, K) for _ in range(cnt)]
            del raw
            for nc in (4, 1):
                xq = torch.randint(-127, 128, (nc * K,), dtype=torch.int8, device=dev, generator=g)
                xd = torch.rand(nc * K // 32, device=dev, generator=g) * 0.01
                y = torch.empty(nc * N, device=dev)
                it = iter(range(1 << 30))  # the graph's nodes walk the matrices
                us = time_graph(torch, lambda: (lambda i: q27.ops.qgemv(mats[i % cnt], xq, xd, y, nc))(next(it)), cnt)
                b = nbytes + nc * K * (1 + 4 / 32) + nc * N * 4
                res[f"{N}x{K}_T{nc}"] = {"us": round(us, 2), "GBps": round(b / us / 1e3, 1),
                                         "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 3), "matrix_MB": round(nbytes / 1e6, 2)}
                log(f"  gemv {name:6s} {N:6d}x{K:<6d} T={nc} {us:7.2f} us {b / us / 1e3:7.1f} GB/s")
            del mats
            torch.cuda.empty_cache()
        out[name] = res
    return out


def bench_fused_gemv(q27, torch):
    """quantize_q8_1 + qgemv (two launches, src/model.cu:727-728 and 826-827) against q27h_qgemv_f32 (one launch) at the
    decode shapes where the reference quantizes separately: the attention output projection (5120 x 6144) and the MTP
    concat projection (5120 x 10240), T = 4, IQ3_S and Q4_K weights. Each timed graph holds 24 pairs (or 24 fused
    launches) over 24 distinct matrices, so the weights come from HBM as in a decode step; median replay / 24."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(19)
    out = {}
    for name, (tid, bb, doffs) in (("iq3_s", GEMV_TYPES["iq3_s"]), ("q4_k", GEMV_TYPES["q4_k"])):
        for N, K in ((5120, 6144), (5120, 10240)):
            nc, cnt = 4, 24
            raw = torch.randint(0, 256, (N * (K // 256), bb), dtype=torch.uint8, device=dev, generator=g)
            for off in doffs:
                d = torch.exp2(torch.rand(raw.shape[0], device=dev, generator=g) * 6 - 10).to(torch.float16)
                raw[:, off:off + 2] = d.view(torch.uint8).view(-1, 2)
            mats = [q27.ops.qmat_upload(raw.reshape(-1), tid, N, K) for _ in range(cnt)]
            del raw
            x = torch.randn(nc * K, device=dev, generator=g)
            xq = torch.empty(nc * K, dtype=torch.int8, device=dev)
            xd = torch.empty(nc * K // 32, device=dev)
            y = torch.empty(nc * N, device=dev)
            it = {"i": 0}

            def pair():
                m = mats[it["i"] % cnt]
                it["i"] += 1
                q27.ops.quantize_q8_1(x, xq, xd, K, nc)
                q27.ops.qgemv(m, xq, xd, y, nc)

            def fused():
                m = mats[it["i"] % cnt]
                it["i"] += 1
                q27.ops.qgemv_f32(m, x, y, nc)

            us_pair = time_graph(torch, pair, cnt)
            us_fused = time_graph(torch, fused, cnt)
            out[f"{name}_{N}x{K}_T{nc}"] = {"unfused_us": round(us_pair, 2), "fused_us": round(us_fused, 2)}
            log(f"  quantize+qgemv {name} {N}x{K} T={nc}: {us_pair:6.2f} us as two launches, {us_fused:6.2f} us fused")
            del mats
            torch.cuda.empty_cache()
    return out


def bench_gdn(q27, torch, M=2048):
    """The delta-rule recurrence (gdn_step, src/ops.cu:449-572) of one GDN layer at the model's head counts (48
    value heads on 16 key heads, 128 x 128 f32 state each): prefill of M tokens in flip mode (the chunked form on
    matrix cores, and the sequential bit-exact kernel beside it) and a decode launch of T = 4 tokens with snapshots
    (graph-replayed, as in a decode step). GB/s counts the compulsory bytes: state in
    and out (plus the snapshot planes), q / k per key head, v, g, beta and o per token. The recurrence is serial in
    the tokens, so its bound is the per-token latency of the update chain, not HBM; us_per_token reports that."""
    dev = torch.device("cuda:0")
    H, HK, D = 48, 16, 128
    stride = 2 * HK * D + H * D
    g = torch.Generator(device=dev)
    g.manual_seed(17)
    out = {}
    for name, T, flip in (("prefill", M, True), ("decode_T4", 4, False)):
        x = torch.randn(T * stride, device=dev, generator=g) * 0.088
        gg = -torch.rand(T * H, device=dev, generator=g) * 0.5
        beta = torch.rand(T * H, device=dev, generator=g)
        planes = torch.randn(4 * H * D * D, device=dev, generator=g) * 0.5
        pin = torch.zeros(1, dtype=torch.int32, device=dev)
        o = torch.empty(T * H * D, device=dev)

        def fn(i=0):
            q27.ops.gdn_step(x, x[HK * D:], x[2 * HK * D:], stride, gg, beta, planes, pin, o, H, HK, T, 0.0884, not flip,
                             flip=flip)

        us = time_back_to_back(torch, fn, 20) if flip else time_graph(torch, fn, 64)
        state = H * D * D * 4
        b = state * (1 + (1 if flip else T)) + T * (2 * HK * D + 2 * H * D + 2 * H) * 4
        out[name] = {"us": round(us, 2), "tokens": T, "us_per_token": round(us / T, 3), "GBps": round(b / us / 1e3, 1),
                     "MB": round(b / 1e6, 2)}
        log(f"  gdn_step {name:9s} T={T:5d} {us:8.2f} us ({us / T:.3f} us/token) {b / us / 1e3:7.1f} GB/s")
        if flip:  # the same prefill on the sequential, bit-exact kernel
            prev = q27.ops.gdn_prefill_exact(True)
            us_seq = time_back_to_back(torch, fn, 20)
            q27.ops.gdn_prefill_exact(prev)
            out[name + "_sequential"] = {"us": round(us_seq, 2), "tokens": T, "us_per_token": round(us_seq / T, 3),
                                         "GBps": round(b / us_seq / 1e3, 1)}
            # multiply-adds of the three state products (K S, Q S, K^T Delta) per token and head, fp32 matrix cores
            out[name]["state_products_TFLOPs"] = round(3 * 2 * D * D * T * H / (us * 1e-6) / 1e12, 2)
            # the same as a share of the dense fp32 matrix-core peak (157.3 TFLOP/s)
            out[name]["state_products_frac_fp32_mfma_peak"] = round(out[name]["state_products_TFLOPs"] / 157.3, 4)
            log(f"  gdn_step {name + '_sequential':9s} T={T:5d} {us_seq:8.2f} us ({us_seq / T:.3f} us/token)")
    return out


def bench_upload(q27, torch, gib=1.0):
    """Weight upload from a GGUF file (the reader of src/gguf.cpp and the transfer of src/qmat.h:34): a file of
    IQ3_S matrices (17408 x 5120 each) written to a temporary directory and mapped, then every tensor copied to HBM
    (a) with q27h_gguf_upload_rows (pread by 8 threads into pinned staging buffers, DMA overlapped), (b) with
    q27h_copy_h2d_staged from the mapping, and (c) as the reference does it, one host-to-device copy from the
    pageable mapping (torch's copy_ of the mapped bytes). Both read the file from the
    page cache (it was just written). Best of 3 passes, GB/s of file bytes."""
    import tempfile

    import numpy as np

    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests"))
    import gguf_writer as W

    dev = torch.device("cuda:0")
    N, K = 17408, 5120
    tb = N * K // 256 * 110
    count = max(1, int(gib * (1 << 30) // tb))
    r = np.random.default_rng(3)
    blob = r.integers(0, 256, tb, dtype=np.uint8).tobytes()
    out = {}
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "w.gguf")
        with open(path, "wb") as f:
            f.write(W.build([("general.architecture", W.STR, "qwen35")],
                            [(f"blk.{i}.ffn_up.weight", 21, (K, N), blob) for i in range(count)]))
        t0 = time.perf_counter()
        g = q27.gguf.GGUF(path)
        parse_ms = (time.perf_counter() - t0) * 1e3
        ts = g.tensors()
        dst = torch.empty(tb, dtype=torch.uint8, device=dev)
        total = tb * count
        for name, fn in (("staged_pread", lambda t: q27.gguf.upload_rows(t, dst, threads=8)),
                         ("staged_from_mapping", lambda t: q27.gguf.copy_h2d_staged(dst, t.data, t.nbytes, threads=8)),
                         ("pageable_copy", lambda t: dst.copy_(torch.from_numpy(t.array()), non_blocking=False))):
            best = 1e9
            for _ in range(3):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for t in ts:
                    fn(t)
                torch.cuda.synchronize()
                best = min(best, time.perf_counter() - t0)
            out[name] = {"GBps": round(total / best / 1e9, 2), "s": round(best, 3)}
            log(f"  upload {name:14s} {total / 1e9:.2f} GB in {best * 1e3:.0f} ms: {total / best / 1e9:.2f} GB/s")
        g.close()
    out.update({"file_GB": round(total / 1e9, 2), "tensors": count, "parse_ms": round(parse_ms, 3)})
    return out


def bench_repack(q27, torch, N=17408, K=5120):
    """The repack of qmat_upload (src/qmat.h:34-36) for each weight type at 17408 x 5120: raw GGUF rows already in
    HBM (random bytes: the repack only moves bytes), two raw copies alternated so the MALL does not serve the input;
    mean of 10 launches. GB/s of raw bytes read + repacked bytes written."""
    dev = torch.device("cuda:0")
    out = {}
    for name, (tid, bb, _) in GEMV_TYPES.items():
        raw_bytes = N * K // 256 * bb
        nbytes = q27.ops.qmat_bytes(tid, N, K)
        raws = [torch.randint(0, 256, (raw_bytes,), dtype=torch.uint8, device=dev) for _ in range(2)]
        buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        st = torch.cuda.current_stream().cuda_stream
        L = q27.ops.lib()
        for i in range(2):
            q27.ops.check(L.q27h_qmat_repack(tid, N, K, raws[i].data_ptr(), buf.data_ptr(), st))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = 10
        torch.cuda.synchronize()
        e0.record()
        for i in range(n):
            q27.ops.check(L.q27h_qmat_repack(tid, N, K, raws[i % 2].data_ptr(), buf.data_ptr(), st))
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / n
        out[name] = {"us": round(us, 2), "raw_MB": round(raw_bytes / 1e6, 1),
                     "GBps": round((raw_bytes + nbytes) / us / 1e3, 1)}
        log(f"  repack {name:8s} {N} x {K}: {us:8.2f} us, {(raw_bytes + nbytes) / us / 1e3:7.1f} GB/s")
        del raws, buf
    return out


def bench_bf16_pair(q27, torch, N=HV, K=E):
    """gemv_bf16_pair (src/ops.h:24-26), the decode alpha / beta projections: ya = Wa x, yb = Wb x for two bf16 [48][5120]
    matrices at T = 1 and 4 tokens. `graph`: launches replayed from one HIP graph on one weight pair (decode-sized,
    as in a decode step's graph; the 0.98 MB pair stays in the caches); `cold`: a graph whose nodes walk 320 weight
    pairs (315 MB, more than the 256 MB MALL), as each GDN layer of a decode step reads its own. GB/s of the weights,
    x and y per launch."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(37)
    sets = 320
    W = [(torch.randint(0, 65536, (N * K,), dtype=torch.int32, device=dev, generator=g).to(torch.int16),
          torch.randint(0, 65536, (N * K,), dtype=torch.int32, device=dev, generator=g).to(torch.int16)) for _ in range(sets)]
    for wa, wb in W:  # finite bf16 weights: clear the top exponent bit
        wa &= 0x3FFF
        wb &= 0x3FFF
    out = {}
    for T in (1, 4):
        x = torch.randn(T * K, device=dev, generator=g)
        ya, yb = torch.empty(T * N, device=dev), torch.empty(T * N, device=dev)
        b = 2 * N * K * 2 + T * K * 4 + 2 * T * N * 4
        us_g = time_graph(torch, lambda: q27.ops.gemv_bf16_pair(W[0][0], W[0][1], x, ya, yb, N, K, T), 200)
        it = iter(range(1 << 30))  # the graph's nodes walk the weight pairs
        us_c = time_graph(torch, lambda: (lambda i: q27.ops.gemv_bf16_pair(W[i % sets][0], W[i % sets][1], x, ya, yb, N,
                                                                           K, T))(next(it)), sets)
        out[f"T{T}"] = {"graph_us": round(us_g, 2), "cold_us": round(us_c, 2), "cold_GBps": round(b / us_c / 1e3, 1),
                        "MB": round(b / 1e6, 2)}
        log(f"  gemv_bf16_pair T={T}: {us_g:.2f} us in a graph, {us_c:.2f} us cold ({b / us_c / 1e3:.0f} GB/s)")
    del W
    torch.cuda.empty_cache()
    return out


def bench_wire(q27, torch, M=2048):
    """The two-card wire formats at the prefill batch (src/prefill.cu:338-406) on one GPU: to_q8_wire with carried
    error feedback, add_norm_rows_q8 (h = null, xs) and to_bf16 of [M][5120], both q8 widths. Three buffer sets
    are cycled; GB/s of the algorithmic bytes per launch."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(31)
    out = {}
    sets = 3
    for qb in (16, 32):
        rb = E + 2 * E // qb
        p = [torch.randn(M * E, device=dev, generator=g) for _ in range(sets)]
        ef = [torch.zeros(M * E, device=dev) for _ in range(sets)]
        wire = [torch.zeros(M * rb, dtype=torch.uint8, device=dev) for _ in range(sets)]
        for i in range(sets):
            q27.ops.to_q8_wire(p[i], ef[i], True, wire[i], E, M, qb=qb)
        us = time_back_to_back(torch, lambda i: q27.ops.to_q8_wire(p[i % sets], ef[i % sets], False, wire[i % sets], E, M,
                                                                   qb=qb), 30)
        b = M * (E * 4 * 2 + rb + E * 4)  # partial + ef in, wire + ef out
        out[f"to_q8_wire_qb{qb}"] = {"us": round(us, 2), "GBps": round(b / us / 1e3, 1), "MB": round(b / 1e6, 1)}
        x = [torch.randn(M * E, device=dev, generator=g) for _ in range(sets)]
        w = torch.randn(E, device=dev, generator=g) * 0.1 + 1
        xq, xd, xs = torch.empty(M * E, dtype=torch.int8, device=dev), torch.empty(M * E // 32, device=dev), torch.empty(
            M * E // 16, device=dev)
        us = time_back_to_back(torch, lambda i: q27.ops.add_norm_rows_q8(x[i % sets], wire[i % sets], wire[(i + 1) % sets], E,
                                                                         M, w, EPS, None, xq, xd, xs, qb=qb), 30)
        b = M * (E * 4 * 2 + 2 * rb + E + E // 32 * 4 + E // 16 * 4) + E * 4
        out[f"add_norm_rows_q8_qb{qb}"] = {"us": round(us, 2), "GBps": round(b / us / 1e3, 1), "MB": round(b / 1e6, 1)}
        log(f"  wire qb={qb}: to_q8_wire {out[f'to_q8_wire_qb{qb}']['us']} us, add_norm_rows_q8 "
            f"{out[f'add_norm_rows_q8_qb{qb}']['us']} us")
        del p, ef, wire, x
    xs_ = [torch.randn(M * E, device=dev, generator=g) for _ in range(sets)]
    y = torch.empty(M * E, dtype=torch.int16, device=dev)
    us = time_back_to_back(torch, lambda i: q27.ops.to_bf16(xs_[i % sets], y, M * E), 30)
    b = M * E * 6
    out["to_bf16"] = {"us": round(us, 2), "GBps": round(b / us / 1e3, 1), "MB": round(b / 1e6, 1)}
    log(f"  wire: to_bf16 {us:.2f} us")
    torch.cuda.empty_cache()
    return out


def bench_decode_graph(q27, torch, replays):
    """The decode verify pass (T = 4): its launches recorded in one HIP graph, median replay time over `replays`
    replays, then the per-op node costs."""
    Dp = Pass(q27, torch, 4, decode=True)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        Dp.run()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            Dp.run()
    torch.cuda.synchronize()
    for _ in range(5):
        graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(replays):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b) * 1e3)
    times.sort()
    decode_us = times[len(times) // 2]
    log(f"decode verify pass: {len(Dp.launches)} launches in one graph, median {decode_us:.1f} us")
    del graph
    decode_ops = bench_decode_ops(q27, torch, Dp)
    del Dp
    torch.cuda.empty_cache()
    return decode_us, decode_ops


def bench_isolated(q27, torch, P, reps=3):
    """Every prefill op alone: all of its launches of the cold pass back to back between two HIP events (distinct
    inputs per launch, so the MALL does not serve them: 48-128 launches of 42-285 MB each), best of `reps` rounds.
    Launched from the host (the shortest, the gather, takes 8.5 us on the GPU, above the host's launch interval; a
    graph adds about 1.5 us per node here: 10.1 us).
    rmsnorm_q8 and the gather run once per pass; they are cycled over the 8 residual buffers instead."""
    o, M = q27.ops, P.M
    groups = {}
    for name, b, fn in P.launches:
        groups.setdefault(name, []).append((b, fn))
    xsq = None if P.decode else P.xs
    groups["rmsnorm_q8"] = [(bytes_rmsnorm_q8(M, True, True),
                             lambda x=x: o.rmsnorm_q8(x, P.norm_w[0], P.h, P.xq, P.xd, E, M, EPS, None, xsq)) for x in P.xs_ring]
    groups["get_rows_iq2_s"] = [(bytes_get_rows(M, P.uniq, P.row_bytes),
                                 lambda x=x: o.get_rows_iq2_s(P.table, P.row_bytes, P.ids, M, x, E)) for x in P.xs_ring]
    # the two sum_norm_rows of a layer share the residual x: run all first ones, then all second ones, so that no
    # launch finds x in the MALL from the launch before it
    groups["sum_norm_rows"] = groups["sum_norm_rows"][0::2] + groups["sum_norm_rows"][1::2]
    out = {}
    for name, L in groups.items():
        for _, fn in L[:3]:
            fn()
        best = 1e30
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _, fn in L:
                fn()
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b) * 1e3)
        nb = sum(b for b, _ in L)
        us = best / len(L)
        gbs = nb / (best * 1e-6) / 1e9
        out[name] = {"us": round(us, 2), "GBps": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 3),
                     "launches": len(L), "bytes_per_launch": nb // len(L)}
        log(f"  isolated {name:18s} {us:8.2f} us  {gbs:8.1f} GB/s ({gbs / HBM_PEAK_GBS:.1%}) over {len(L)} launches")
    P.reset()
    return out


def bench_cfg1(q27, torch):
    """RMSNorm -> q8_1 of one 5120 row (0.1% outliers x50) on the CPU oracle and on the GPU, with the
    bit-exact comparison of xq / xd / xs."""
    import numpy as np

    sys.path.insert(0, ROOT)
    from oracle import q27_oracle as O

    r = np.random.default_rng(1)
    x = r.standard_normal(E).astype(np.float32)
    x[r.choice(E, 5, replace=False)] *= 50
    w = (r.standard_normal(E) * 0.1 + 1).astype(np.float32)
    t0 = time.perf_counter()
    for _ in range(200):
        _, oq, od, os_ = O.rmsnorm_q8(x, w, E, 1, EPS, with_h=False, with_xs=True)
    cpu_us = (time.perf_counter() - t0) / 200 * 1e6
    dx, dw = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    xq = torch.empty(E, dtype=torch.int8, device="cuda")
    xd, xs = torch.empty(E // 32, device="cuda"), torch.empty(E // 16, device="cuda")
    fn = lambda: q27.ops.rmsnorm_q8(dx, dw, None, xq, xd, E, 1, EPS, None, xs)  # noqa: E731
    gpu_us = time_graph(torch, fn, 50)
    exact = (np.array_equal(xq.cpu().numpy(), oq) and np.array_equal(xd.cpu().numpy().view(np.uint32), od.view(np.uint32))
             and np.array_equal(xs.cpu().numpy().view(np.uint32), os_.view(np.uint32)))
    log(f"  cfg1 rmsnorm_q8 1x5120: cpu oracle {cpu_us:.1f} us (1 thread), gpu {gpu_us:.2f} us, bit-exact {exact}")
    return {"cpu_us_1thread": round(cpu_us, 2), "gpu_us_graph": round(gpu_us, 2), "bytes": 48000, "bit_exact": bool(exact)}


def bench_decode_ops(q27, torch, Dp):
    """configs[1] per op: median time per launch with 50 launches of the op replayed from one HIP graph."""
    res = {}
    seen = set()
    for name, b, fn in Dp.launches:
        if name in seen:
            continue
        seen.add(name)
        us = time_graph(torch, fn, 50)
        res[name] = {"us": round(us, 2), "bytes": b}
        log(f"  decode {name:18s} {us:6.2f} us per launch (graph)")
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--graph-replays", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline")
    ap.add_argument("--cpu-rows", type=int, default=4096)
    ap.add_argument("--gemv-profile", default=None, metavar="TYPE,N,K,T",
                    help="only run eight decode GEMV launches of this shape over four uploaded copies of a random "
                         "matrix (the workload of the rocprofv3 counter runs of the GEMV), then exit")
    ap.add_argument("--calib-copy", action="store_true", help="also run a plain 256 MiB copy (rocprof counter calibration)")
    ap.add_argument("--buffers", choices=("cold", "warm"), default="cold",
                    help="prefill step inputs: cold = every layer reads its own (default), warm = one set reused by all layers")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the timed prefill steps (for rocprof counter runs): no breakdown, roofline, decode or CPU legs")
    ap.add_argument("--repack-only", action="store_true", help="only the qmat_upload repack of each weight type")
    ap.add_argument("--decode-only", action="store_true", help="only the decode verify pass (T = 4) graph")
    ap.add_argument("--cfg45-only", action="store_true",
                    help="only the configs[3] gathers and the configs[4] multimodal legs (for rocprof counter runs)")
    ap.add_argument("--isolated-only", action="store_true",
                    help="only the per-op isolated legs of the prefill pass (each op's launches back to back)")
    ap.add_argument("--gdn-only", action="store_true", help="only the delta-rule recurrence legs (for rocprof counter runs)")
    ap.add_argument("--wire-only", action="store_true", help="only the gemv_bf16_pair and two-card wire-format legs")
    ap.add_argument("--gemv-only", action="store_true", help="only the decode GEMV legs (every weight type)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the fused-op path has no multi-GPU form in this build "
              "(sharding by token rows needs no exchange). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.gemv_profile:
        gemv_profile(*[int(v) for v in args.gemv_profile.split(",")])
        return

    import torch

    q27 = load_package()
    q27.lib()
    torch.cuda.init()
    log(f"device: {torch.cuda.get_device_name(0)}")
    if args.repack_only:
        print(json.dumps({"qmat_repack": bench_repack(q27, torch)}), flush=True)
        return
    if args.cfg45_only:
        out = {"gathers_cfg4": bench_gathers(q27, torch)}
        torch.cuda.empty_cache()
        out["multimodal_cfg5"] = bench_multimodal(q27, torch)
        print(json.dumps(out), flush=True)
        return
    if args.decode_only:
        decode_us, decode_ops = bench_decode_graph(q27, torch, args.graph_replays)
        print(json.dumps({"decode_us_per_step": round(decode_us, 1), "decode_per_op": decode_ops}), flush=True)
        return
    if args.gdn_only:
        print(json.dumps({"gdn_recurrence": bench_gdn(q27, torch)}), flush=True)
        return
    if args.gemv_only:
        print(json.dumps({"decode_gemv": bench_gemv(q27, torch)}), flush=True)
        return
    if args.wire_only:
        print(json.dumps({"gemv_bf16_pair": bench_bf16_pair(q27, torch), "wire_formats": bench_wire(q27, torch)}),
              flush=True)
        return

    # ---- prefill pass (the step)
    P = Pass(q27, torch, 2048, decode=False, cold=args.buffers == "cold")
    if args.isolated_only:
        for _ in range(args.warmup):
            P.run()
        torch.cuda.synchronize()
        print(json.dumps({"per_op_isolated": bench_isolated(q27, torch, P)}), flush=True)
        return
    step_bytes = P.bytes_per_step()
    log(f"prefill pass: {len(P.launches)} launches, {step_bytes / 1e9:.3f} GB algorithmic per step")
    for _ in range(args.warmup):
        P.reset()
        P.run()
    torch.cuda.synchronize()
    P.reset()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        P.run()
    e1.record()
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"prefill: {ms_per_step * 1e3:.1f} us per 2048-token batch, {value:.0f} GB/s")
    if args.prefill_only:
        if args.calib_copy:
            src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
            dst = torch.empty_like(src)
            for _ in range(3):
                dst.copy_(src)
            torch.cuda.synchronize()
            log("calibration copy: 3 x 256 MiB device-to-device")
        print(json.dumps({"metric": "prefill-only profiling run", "value": round(value, 1), "unit": "GB/s",
                          "ms_per_step": round(ms_per_step, 4)}), flush=True)
        return

    # ---- per-op breakdown inside the pass (HIP events around each launch)
    acc = {}
    for _ in range(max(1, min(3, args.steps))):
        P.run_events(acc)
    # An event pair around every launch adds a fixed cost per launch (the kernel waits behind the event marker).
    # It is estimated as (sum of the per-launch event times - the pass time without events) / launches and
    # subtracted in "net_us"; the rocprof kernel durations in profiles/ are the direct measurement.
    npass = max(1, min(3, args.steps))
    ev_total_us = sum(ms for ms, _, _ in acc.values()) * 1e3 / npass
    n_launch = sum(cnt for _, cnt, _ in acc.values()) // npass
    ev_overhead_us = max(0.0, (ev_total_us - ms_per_step * 1e3) / n_launch)
    log(f"event-pair overhead: {ev_overhead_us:.2f} us per launch")
    per_op = {}
    for name, (ms, cnt, b) in acc.items():
        us = ms * 1e3 / cnt
        net = max(us - ev_overhead_us, 1e-3)
        gbs = (b / cnt) / (us * 1e-6) / 1e9
        gbs_net = (b / cnt) / (net * 1e-6) / 1e9
        per_op[name] = {"us": round(us, 2), "GBps": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 3),
                        "net_us": round(net, 2), "net_GBps": round(gbs_net, 1),
                        "net_hbm_frac": round(gbs_net / HBM_PEAK_GBS, 3),
                        "bytes": b // cnt, "launches_per_step": cnt // npass}
        log(f"  {name:18s} {us:9.2f} us  {gbs:8.1f} GB/s  ({gbs / HBM_PEAK_GBS:.1%} of 8 TB/s); "
            f"net {net:7.2f} us ({gbs_net / HBM_PEAK_GBS:.1%})")
    # ---- each op alone (MALL-proof), and the pass with one set of buffers reused by every layer (warm)
    isolated = bench_isolated(q27, torch, P)
    Pw = Pass(q27, torch, 2048, decode=False, cold=False)
    for _ in range(2):
        Pw.run()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(args.steps):
        Pw.run()
    b.record()
    torch.cuda.synchronize()
    warm_us = a.elapsed_time(b) * 1e3 / args.steps
    log(f"prefill pass with one buffer set for all layers (MALL-warm): {warm_us:.1f} us")
    del Pw
    # ---- roofline of the dominant kernel (swiglu_q8 at M = 2048): its 64 launches of the cold pass back to back
    # between two HIP events on the stream the kernel runs on (torch's current stream, which the launchers use);
    # every launch reads its own 285 MB of g, u, so none is served by the MALL
    sw = isolated["swiglu_q8"]
    sw_us, sw_bytes = sw["us"], sw["bytes_per_launch"]
    sw_gbs = sw_bytes / (sw_us * 1e-6) / 1e9
    log(f"swiglu_q8 back-to-back: {sw_us:.2f} us per launch, {sw_gbs:.0f} GB/s")
    roofline = {"bound": "hbm", "achieved": round(sw_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(sw_gbs / HBM_PEAK_GBS, 4), "traffic": SWIGLU_TRAFFIC_BYTES, "kernel": "swiglu_q8 (flat_q8_kernel<true>)",
                "bytes_per_launch": sw_bytes, "avg_launch_us": round(sw_us, 2),
                "note": "2048 x 17408 values, 9.375 B each (g, u f32 in; xq int8, xd f32 per 32, xs f32 per 16 out)"}
    # sum_norm_rows takes as long per pass as swiglu_q8 (128 launches of half the time); its isolated figure beside it
    sn = isolated["sum_norm_rows"]
    roofline["co_dominant"] = {"kernel": "sum_norm_rows (row_norm_q8_kernel<1>)", "achieved": sn["GBps"],
                               "frac": round(sn["GBps"] / HBM_PEAK_GBS, 4), "avg_launch_us": sn["us"],
                               "bytes_per_launch": sn["bytes_per_launch"], "launches_per_pass": sn["launches"]}
    # ---- practical copy ceiling of this device (torch device-to-device copy of 512 MiB, read + write bytes)
    src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    a.record()
    for _ in range(10):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    copy_gbs = 2 * (512 << 20) * 10 / (a.elapsed_time(b) * 1e-3) / 1e9
    log(f"device copy ceiling: {copy_gbs:.0f} GB/s")
    del src, dst, P
    torch.cuda.empty_cache()

    # ---- decode verify pass (T = 4) in one HIP graph
    decode_us, decode_ops = bench_decode_graph(q27, torch, args.graph_replays)

    # ---- configs[0], configs[3] (gathers) and configs[4] (multimodal + GDN)
    cfg1 = bench_cfg1(q27, torch)
    gathers = bench_gathers(q27, torch)
    torch.cuda.empty_cache()
    multimodal = bench_multimodal(q27, torch)
    torch.cuda.empty_cache()
    gemv = bench_gemv(q27, torch)
    torch.cuda.empty_cache()
    fused_gemv = bench_fused_gemv(q27, torch)
    gdn_rec = bench_gdn(q27, torch)
    pair = bench_bf16_pair(q27, torch)
    wire = bench_wire(q27, torch)
    upload = bench_upload(q27, torch)
    repack = bench_repack(q27, torch)

    if args.calib_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration copy: 3 x 256 MiB device-to-device")

    cpu = None
    if not args.no_cpu:
        hw = host_cpu_info()
        # the pool gives each GPU a share of 16 host cores (its OMP_NUM_THREADS); use all of that share
        share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or hw["affinity_cpus"]
        threads = max(1, min(share, hw["affinity_cpus"]))
        sh = _cpu_shared()
        cpu_ops = {}
        gbs1, secs1 = cpu_baseline(max(1, args.cpu_rows // threads), 1, sh, cpu_ops)
        gbsn, secsn = cpu_baseline(args.cpu_rows, threads, sh)
        cpu = {"value": round(gbsn, 3), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": (f"the prefill pass (64 layers, 322 launches of the oracle) on {args.cpu_rows} token rows split over "
                          f"{threads} threads ({args.cpu_rows // threads} rows each, Zipf ids into the full 248320-row IQ2_S "
                          f"table, q8_0 cache of 180224 rows at pos0 131072): {secsn:.1f} s; single thread on "
                          f"{max(1, args.cpu_rows // threads)} rows: {gbs1:.3f} GB/s ({secs1:.1f} s)"),
               "single_thread_GBps": round(gbs1, 3),
               "single_thread_per_op": {k: {"GBps": round(b / t / 1e9, 3), "s": round(t, 3)} for k, (t, b) in cpu_ops.items()},
               "host": hw,
               "us_per_2048_batch_equiv": round(step_bytes / (gbsn * 1e9) * 1e6, 0)}
        log(f"cpu oracle: {gbsn:.3f} GB/s on {threads} threads ({secsn:.1f} s), {gbs1:.3f} GB/s on 1 thread ({secs1:.1f} s); {hw}")

    out = {
        "metric": "achieved HBM GB/s of the fused per-layer ops over one 2048-token prefill pass",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded; random weights of the Qwen3.8-27B layer shapes)",
        "config": {"workload": "configs[2]: prefill batch of 2048 tokens, 64 layers of in-scope launches "
                               "(48 GDN + 16 attention), q8_0 KV cache of 180224 rows, IQ2_S embedding",
                   "tokens": 2048, "layers": N_LAYER, "launches_per_step": len(acc) and sum(v["launches_per_step"] for v in per_op.values())},
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "copy_ceiling_GBps": round(copy_gbs, 1),
        "us_per_2048_batch": round(ms_per_step * 1e3, 1),
        "decode_us_per_step": round(decode_us, 1),
        "us_per_2048_batch_warm": round(warm_us, 1),
        "per_op": per_op,
        "per_op_isolated": isolated,
        "per_op_event_overhead_us": round(ev_overhead_us, 2),
        "decode_per_op": decode_ops,
        "cfg1_rmsnorm_q8_row": cfg1,
        "gathers_cfg4": gathers,
        "multimodal_cfg5": multimodal,
        "decode_gemv": gemv,
        "decode_quantize_gemv_fused": fused_gemv,
        "gdn_recurrence": gdn_rec,
        "gemv_bf16_pair": pair,
        "wire_formats": wire,
        "gguf_upload": upload,
        "qmat_repack": repack,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
