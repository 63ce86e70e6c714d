"""The measurement probes (probe.hip) that bench.py reports as practical
peaks, each run once at a small size: every kind of rlq_probe_mfma and every
launch shape of rlq_probe_stream_shape returns RLQ_OK, completes, writes the
words it documents and nothing past them.  The MFMA probes run twice on
output buffers filled differently beforehand: a word they write is the same
deterministic value both times.  The stream probes' words are checked
against the XOR of each wave's runs recomputed on the host.  Every test
prints its case before touching the GPU.
"""
import ctypes

import numpy as np
import pytest

from rlq_loader import load

pytestmark = pytest.mark.gpu

rlq = load()
torch = rlq.torch


def say(*a):
    print("[case]", *a, flush=True)


def stream_ptr():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def probe_words(kind, wgs):
    """(words per workgroup, the indices the probe writes)."""
    if kind < 4:
        return 4, list(range(4 * wgs))
    if kind in (4, 7):  # the FMA waves (4-7) exit
        return 8, [8 * g + w for g in range(wgs) for w in range(4)]
    if kind == 5:  # the MFMA waves (0-3) exit
        return 8, [8 * g + w for g in range(wgs) for w in range(4, 8)]
    return 8, list(range(8 * wgs))


@pytest.mark.parametrize("kind", range(9))
def test_probe_mfma_kinds(kind):
    say("rlq_probe_mfma kind", kind, "2 workgroups, 8 iterations")
    wgs = 2
    per, idx = probe_words(kind, wgs)
    runs = []
    for fill in (-1, 7):
        out = torch.full((per * wgs + 16,), fill, dtype=torch.int32, device="cuda")
        assert rlq.lib().rlq_probe_mfma(kind, wgs, 8, ctypes.c_void_p(out.data_ptr()), stream_ptr()) == 0
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert (got[per * wgs:] == fill).all()  # nothing past the documented words
        runs.append(got)
    assert np.array_equal(runs[0][idx], runs[1][idx])


@pytest.mark.parametrize("waves", [4, 8, 16])
@pytest.mark.parametrize("runs", [1, 2, 4, 8])
@pytest.mark.parametrize("nt", [0, 1])
def test_probe_stream_shapes(waves, runs, nt):
    say("rlq_probe_stream_shape waves", waves, "runs", runs, "nt", nt, "3 workgroups, 200 KB")
    nbytes, wgs = 200 * 1024, 3
    buf = torch.arange(nbytes // 4, dtype=torch.int32, device="cuda")
    out = torch.full((wgs * waves + 16,), -1, dtype=torch.int32, device="cuda")
    rc = rlq.lib().rlq_probe_stream_shape(ctypes.c_void_p(buf.data_ptr()), nbytes, wgs, waves, runs, nt,
                                          ctypes.c_void_p(out.data_ptr()), stream_ptr())
    assert rc == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32)
    assert (got[wgs * waves:] == 0xFFFFFFFF).all()
    # workgroup g reads runs [g per, (g + 1) per) of 1 KB, wave w every waves-th
    # of them from the share's run w; lane l XORs the four words of its 16
    # bytes, and lanes l and l + 32 are folded before lane 0 stores
    data = buf.cpu().numpy().view(np.uint32).reshape(-1, 64, 4)
    lane_x = np.bitwise_xor.reduce(data, axis=2)  # [run][lane]
    total = nbytes // 1024
    per = -(-total // wgs)
    for g in range(wgs):
        r0, r1 = g * per, min(g * per + per, total)
        for w in range(waves):
            x = np.bitwise_xor.reduce(lane_x[r0 + w:r1:waves], axis=0) if r0 + w < r1 else np.zeros(64, np.uint32)
            assert got[g * waves + w] == (x[0] ^ x[32]), (g, w)
