"""GPU side of the GGUF path: the staged host -> HBM copy (q27h_copy_h2d_staged) delivers exactly the file's bytes
(any size, any row range, back-to-back calls reusing the staging buffers, a non-default stream), and a weight
matrix read from a GGUF file, uploaded and repacked gives the oracle's GEMV bit for bit."""
import sys

import numpy as np
import pytest

import cfgdata as cd
import gguf_writer as W
from conftest import assert_bits_equal

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-gguf] {msg}", flush=True)
    sys.stdout.flush()


def test_staged_copy_sizes(q27, dev):
    import torch

    r = np.random.default_rng(1)
    for n in (1, 15, 4096 + 3, (32 << 20) - 1, (32 << 20) + 17, (130 << 20) + 5):
        say(f"staged copy {n} bytes")
        src = r.integers(0, 256, n, dtype=np.uint8)
        dst = torch.zeros(n + 64, dtype=torch.uint8, device=dev)
        q27.gguf.copy_h2d_staged(dst[32:], src.ctypes.data, n)
        torch.cuda.synchronize()
        got = dst.cpu().numpy()
        assert np.array_equal(got[32:32 + n], src) and not got[:32].any() and not got[32 + n:].any()


def test_staged_copy_back_to_back_on_a_stream(q27, dev):
    """Six 40 MiB copies in a row from one reused host buffer (overwritten after each call returns) onto a side
    stream: each device copy holds the bytes the host buffer had during its own call."""
    import torch

    n = 40 << 20
    src = np.empty(n, np.uint8)
    outs = [torch.empty(n, dtype=torch.uint8, device=dev) for _ in range(6)]
    s = torch.cuda.Stream()
    for i, o in enumerate(outs):
        src[:] = i + 1
        src[i * 1000] = 200
        q27.gguf.copy_h2d_staged(o, src.ctypes.data, n, threads=3, s=s.cuda_stream)
    s.synchronize()
    for i, o in enumerate(outs):
        a = o.cpu().numpy()
        assert a[i * 1000] == 200 and np.count_nonzero(a != i + 1) == 1, i


def test_gguf_to_qgemv(q27, oracle, dev, tmp_path):
    """A file holding two weight matrices: rows [8, 1032) of the second uploaded with upload_rows, repacked, and
    multiplied: the oracle's y on the same raw rows, bit for bit."""
    import torch

    r = cd.rng(7)
    N, K = 1040, 2560
    w1 = cd.random_weights(r, cd.Q4_K, 16, 512)
    w2 = cd.random_weights(r, cd.IQ3_S, N, K)
    path = tmp_path / "w.gguf"
    path.write_bytes(W.build([("general.architecture", W.STR, "qwen35")],
                             [("a.weight", cd.Q4_K, (512, 16), w1.tobytes()), ("b.weight", cd.IQ3_S, (K, N), w2.tobytes())]))
    with q27.gguf.GGUF(str(path)) as g:
        t = g.tensor("b.weight")
        assert t.rows() == N and t.row_bytes() == K // 256 * 110
        say("gguf upload + qgemv")
        row0, n = 8, 1024
        raw = torch.empty(n * t.row_bytes(), dtype=torch.uint8, device=dev)
        q27.gguf.upload_rows(t, raw, row0, n)
        m = q27.ops.qmat_upload(raw, t.type, n, K)
        xq, xd = cd.q8_activations(oracle, r, 2, K)
        y = torch.zeros(2 * n, device=dev)
        q27.ops.qgemv(m, torch.from_numpy(xq).to(dev), torch.from_numpy(xd).to(dev), y, 2)
        torch.cuda.synchronize()
        want = oracle.qgemv(cd.IQ3_S, w2.reshape(N, -1)[row0:row0 + n].copy(), n, K, xq, xd, 2)
        assert_bits_equal(y.cpu().numpy().reshape(2, n), want, "gguf -> qgemv")
        with pytest.raises(q27.Q27Error):
            q27.gguf.upload_rows(t, raw, N - 8, 16)
