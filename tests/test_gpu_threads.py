"""Two host threads, each with its own context and stream, driving the
library at once: every output must be bitwise the output of the same calls
made one after another.  The reference's matvec entry points keep no global
state (crates/quant/src/matvec.rs:24-87) and may be called from any thread;
the library's host side keeps per-device launch state (compute-unit counts,
each kernel's dynamic-LDS limit) that the threads share.

The threaded part runs first in a fresh process, so the two threads are the
first to raise the kernels' LDS limits and read the device's compute units
(in the test process earlier tests have already done that)."""
import os
import subprocess
import sys
import threading

import numpy as np
import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from rlq_loader import load  # noqa: E402

# (type, rows, cols, batch): one column at K = 14336 (activation image and
# parked terms above 64 KB of LDS), the K-split kernels at 3 to 8 columns,
# Q6_K and Q8_0 one-column kernels, the K16 split kernel and the prefill GEMM
CASES = [("Q4_K", 4096, 14336, 1), ("Q5_K", 2048, 4096, 3), ("Q4_K", 3000, 4096, 8), ("Q6_K", 1024, 14336, 1),
         ("Q8_0", 4864, 896, 1), ("Q3_K", 2048, 4096, 2), ("Q6_K", 2000, 4096, 5), ("Q4_K", 1024, 4096, 96),
         ("Q2_K", 1500, 2048, 1)]
REPEATS = 3


def _inputs(rlq, seed):
    g = np.random.default_rng(seed)
    out = []
    for i, (t, rows, cols, batch) in enumerate(CASES):
        w = (g.standard_normal(rows * cols) * 0.02).astype(np.float32)
        x = g.standard_normal((batch, cols)).astype(np.float32)
        out.append((rlq.DType[t], rows, cols, w, x))
    return out


def _run(rlq, ctx, cases, stream, start=None):
    """Quantize (the default context) and upload the weights, then REPEATS
    rounds of every matmul on `stream`; returns the outputs as numpy."""
    torch = rlq.torch
    if start is not None:
        start.wait()
    res = []
    with torch.cuda.stream(stream):
        mats = [(rlq.Weights(ctx, t, rlq.quantize(t, w), rows, cols), torch.from_numpy(x).cuda())
                for t, rows, cols, w, x in cases]
        for _ in range(REPEATS):
            ys = [ctx.matmul(W, x, stream=stream) for W, x in mats]
            ctx.sync(stream)
            res.append([y.cpu().numpy() for y in ys])
        for W, _ in mats:
            W.close()
    return res


def child():
    rlq = load()
    torch = rlq.torch
    torch.cuda.set_device(0)
    cases = [_inputs(rlq, 11), _inputs(rlq, 12)]
    ctxs = [rlq.Context(0), rlq.Context(0)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    out, errs = [None, None], []
    start = threading.Barrier(2)

    def work(i):
        try:
            out[i] = _run(rlq, ctxs[i], cases[i], streams[i], start)
        except BaseException as e:  # reported by the main thread
            errs.append(repr(e))

    print("[case] two threads, two contexts:", ", ".join(f"{t} {r}x{c} B={b}" for t, r, c, b in CASES), flush=True)
    th = [threading.Thread(target=work, args=(i,)) for i in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    if errs:
        print("thread error:", errs, flush=True)
        return 1
    print("[case] the same calls, one after another", flush=True)
    serial = rlq.Context(0)
    bad = 0
    for i in range(2):
        ref = _run(rlq, serial, cases[i], torch.cuda.current_stream())[0]
        for rep in range(REPEATS):
            for k, (t, rows, cols, batch) in enumerate(CASES):
                a, b = out[i][rep][k].view(np.int32), ref[k].view(np.int32)
                if not np.array_equal(a, b):
                    bad += 1
                    print(f"mismatch: thread {i} repeat {rep} {t} {rows}x{cols} B={batch}: "
                          f"{int((a != b).sum())} of {a.size} outputs differ", flush=True)
    for c in ctxs + [serial]:
        c.close()
    print("threads ok" if bad == 0 else f"{bad} mismatches", flush=True)
    return 1 if bad else 0


@pytest.mark.gpu
def test_two_threads_two_contexts_match_serial():
    r = subprocess.run([sys.executable, "-u", os.path.abspath(__file__), "child"], capture_output=True, text=True,
                       timeout=300)
    print(r.stdout[-4000:], r.stderr[-4000:])
    assert r.returncode == 0 and "threads ok" in r.stdout


if __name__ == "__main__" and sys.argv[1:] == ["child"]:
    sys.exit(child())
