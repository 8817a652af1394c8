"""GPU parity of the product at prefill widths and of each kernel path
through the C ABI (iq_matmul / iq_matmul_via).

Tolerance: bitwise.  The dispatch (iq_matmul) keeps the reference's
per-lane f32 order at every row count, so each output row equals the
oracle's (the reference's fused kernel restated) bit for bit, and equals a
one-row call on the same row: the reference tiles prefill rows under that
guarantee (src/gguf.rs:493-520) and refuses builds that would break it
(src/gguf.rs:1043-1053).  The fixed paths of iq_matmul_via (the reference's
MultiRowPath, src/gguf.rs:43-62) are held to the same bar; the tile-order
prefill path is tested in test_gpu_prefill.py.
"""
import threading

import numpy as np
import pytest
import torch

from conftest import assert_bitexact
from inferq_amd import _lib
from inferq_amd import qgemm as Q
from inferq_amd import synth as S

pytestmark = pytest.mark.gpu

Q4, Q6, Q8 = S.Q4_K, S.Q6_K, S.Q8_0


@pytest.mark.parametrize("dtype,rows,cols", [
    (Q4, 1024, 2048), (Q6, 512, 2048), (Q8, 512, 2048), (Q4, 300, 4096), (Q6, 200, 512), (Q6, 37, 768),
    (Q8, 45, 96), (Q4, 13, 256),
])
def test_prefill_widths_bitexact_by_default(gpu, oracle, dtype, rows, cols):
    """64, 100 and 256 input rows (past the decode and verify widths) on the
    exact lane-order MFMA tile where it can read the matrix, the lane kernel
    otherwise (Q6_K with an odd block count per row, Q8_0)."""
    rng = np.random.default_rng(rows * 7 + cols + dtype)
    w = S.random_matrix(dtype, rows, cols, rng)
    mat = Q.QuantizedMatrix.upload(w, dtype, rows, cols)
    impl = 1 if oracle.have_avx2() else 0
    for m in (64, 100, 256):
        x = S.normal((m, cols), np.random.default_rng(3000 + m))
        expected = oracle.matmul(dtype, w, rows, cols, x, impl=impl, nthreads=8)
        got = mat.forward(torch.from_numpy(x).to(gpu)).cpu().numpy()
        assert_bitexact(got, expected, f"{S.NAMES[dtype]} [{rows}x{cols}] m={m}")


@pytest.mark.parametrize("dtype,rows,cols", [(Q4, 8192, 2048), (Q4, 2048, 4096), (Q6, 8192, 2048)],
                         ids=["q4k_8192x2048", "q4k_2048x4096", "q6k_8192x2048"])
def test_prefill_full_size_bitexact_by_default(gpu, oracle, dtype, rows, cols):
    """The BASELINE prefill shapes at full size through the dispatch: [256 x
    2048] -> 8192 and [256 x 4096] -> 2048 (Q4_K), and the Q6_K [256 x 2048]
    -> 8192, on the grid the default call launches, against the threaded
    oracle, bit for bit."""
    rng = np.random.default_rng(rows + cols + dtype)
    w = S.random_matrix(dtype, rows, cols, rng)
    mat = Q.QuantizedMatrix.upload(w, dtype, rows, cols)
    x = S.normal((256, cols), np.random.default_rng(4096 + rows))
    expected = oracle.matmul(dtype, w, rows, cols, x, impl=1 if oracle.have_avx2() else 0, nthreads=8)
    got = mat.forward(torch.from_numpy(x).to(gpu)).cpu().numpy()
    assert_bitexact(got, expected, f"{S.NAMES[dtype]} [256 x {cols}] -> {rows}")


@pytest.mark.parametrize("dtype", [Q4, Q6, Q8], ids=["q4k", "q6k", "q80"])
def test_prefill_rows_equal_one_row_calls(gpu, dtype):
    """256 rows in one call equal 256 one-row calls bitwise: prefill never
    changes an output that decode would produce
    (tests/speculative_policy.rs:373-450 in the reference)."""
    rng = np.random.default_rng(90 + dtype)
    cols = 2048
    mat = Q.QuantizedMatrix.upload(S.random_matrix(dtype, 1024, cols, rng), dtype, 1024, cols)
    x = torch.from_numpy(S.normal((256, cols), rng)).to(gpu)
    wide = mat.forward(x).cpu().numpy()
    singles = torch.cat([mat.forward(x[i:i + 1]) for i in range(256)]).cpu().numpy()
    assert_bitexact(wide, singles, f"{S.NAMES[dtype]} 256 rows vs one-row calls")


PATHS = {_lib.PATH_LANES: "lanes", _lib.PATH_GEMV: "gemv", _lib.PATH_LANE_MFMA: "lane-order MFMA"}


def _covers(path, dtype, m):
    if path == _lib.PATH_GEMV:
        return m < 64
    if path == _lib.PATH_LANE_MFMA:
        return dtype in (Q4, Q6)
    return True


@pytest.mark.parametrize("path", list(PATHS), ids=list(PATHS.values()))
@pytest.mark.parametrize("dtype,rows,cols", [(Q4, 256, 2048), (Q4, 90, 4096), (Q6, 130, 4096), (Q6, 70, 2048),
                                             (Q8, 96, 2048)])
def test_each_path_bitexact(gpu, oracle, path, dtype, rows, cols):
    """Every fixed kernel, at row counts the dispatch would not give it,
    returns the oracle's bits; a kernel that does not cover a case says so
    with an error instead of running."""
    rng = np.random.default_rng(path * 100 + dtype)
    w = S.random_matrix(dtype, rows, cols, rng)
    mat = Q.QuantizedMatrix.upload(w, dtype, rows, cols)
    for m in (1, 3, 5, 8, 9, 16, 63, 64, 70):
        x = S.normal((m, cols), np.random.default_rng(4000 + m))
        xt = torch.from_numpy(x).to(gpu)
        if not _covers(path, dtype, m):
            with pytest.raises(Q.QgemmError, match="kernel for"):
                mat.forward_via(xt, path)
            continue
        got = mat.forward_via(xt, path).cpu().numpy()
        assert_bitexact(got, oracle.matmul(dtype, w, rows, cols, x, nthreads=8),
                        f"{PATHS[path]} {S.NAMES[dtype]} m={m}")


def test_unknown_path_is_rejected(gpu):
    mat = Q.QuantizedMatrix.upload(np.zeros(144, np.uint8), Q4, 1, 256)
    with pytest.raises(Q.QgemmError, match="unknown matmul path 9"):
        mat.forward_via(torch.zeros(1, 256, device=gpu), 9)


def test_concurrent_streams_and_threads(gpu):
    """Two host threads, each on its own stream, call the same matrices
    with row counts that keep growing their workspaces: every result equals
    the sequential one bitwise (the workspace is per stream, and its lock
    is held while a call enqueues)."""
    rng = np.random.default_rng(12)
    mats = [Q.QuantizedMatrix.upload(S.random_matrix(dt, 512, 2048, rng), dt, 512, 2048) for dt in (Q4, Q6, Q8)]
    sizes = [1, 9, 40, 70, 130, 2, 200, 17]
    xs = [torch.from_numpy(S.normal((m, 2048), rng)).to(gpu) for m in sizes]
    expected = [[mt.forward(x).cpu().numpy() for x in xs] for mt in mats]
    torch.cuda.synchronize()
    results = {}
    errors = []

    def worker(tid):
        try:
            stream = torch.cuda.Stream()
            out = []
            with torch.cuda.stream(stream):
                for rep in range(3):
                    for j, x in enumerate(xs):
                        mt = mats[(j + tid + rep) % 3]
                        out.append(((j + tid + rep) % 3, j, mt.forward(x)))
            stream.synchronize()
            results[tid] = [(k, j, y.cpu().numpy()) for k, j, y in out]
        except Exception as exc:  # reported by the main thread
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for tid in range(2):
        for k, j, y in results[tid]:
            assert_bitexact(y, expected[k][j], f"thread {tid} matrix {k} m={sizes[j]}")


@pytest.mark.parametrize("dtype,rows,cols,m", [
    (Q4, 8192, 2048, 4), (Q4, 8192, 2048, 8), (Q4, 2048, 4096, 8), (Q6, 40960, 2048, 8), (Q6, 40960, 2048, 1),
    (Q4, 1024, 2048, 64),
])
def test_graph_replays_match_eager_calls(gpu, dtype, rows, cols, m):
    """A dense call captured in a HIP graph (split-K and pair-lane tiles at
    4-8 rows, the GEMV at one row, the 16-row tile at 64) and replayed
    several times, with fresh inputs copied into its buffer and eager calls
    between replays, gives bitwise the eager call's output each time: the
    kernels record no allocation, memset or host copy."""
    rng = np.random.default_rng(rows + m + dtype)
    mat = Q.QuantizedMatrix.upload(S.random_matrix(dtype, rows, cols, rng), dtype, rows, cols)
    xs = [torch.from_numpy(S.normal((m, cols), rng)).to(gpu) for _ in range(3)]
    eager = [mat.forward(x).cpu().numpy() for x in xs]
    x_buf, y_buf = torch.zeros(m, cols, device=gpu), torch.empty(m, rows, device=gpu)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        mat.forward_into(x_buf, y_buf)  # sizes the workspace outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        mat.forward_into(x_buf, y_buf)
    for rep in range(2):
        for i in range(3):
            x_buf.copy_(xs[i])
            graph.replay()
            torch.cuda.synchronize()
            assert_bitexact(y_buf.cpu().numpy(), eager[i], f"replay {rep}.{i} m={m}")
            y = mat.forward(xs[(i + 1) % 3])  # eager work between replays
            torch.cuda.synchronize()
            assert_bitexact(y.cpu().numpy(), eager[(i + 1) % 3], "eager between replays")
