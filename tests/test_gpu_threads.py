"""Concurrent host callers on the GPU (the reference releases the GIL around every kernel and
allows calls from several Python threads, pybind_entry.cpp:966-969; its thread tests run the
kernel table from several threads and require the same bits, test_threads.cpp:168, :280-299).

Each thread has its own stream and staging buffers (runtime.hip); the weight cache is shared.
Every result computed by a thread must equal, bit for bit, the same call made alone."""

import threading

import numpy as np
import pytest

from oracle import oracle as o
from tests import gpu_util as g

pytestmark = pytest.mark.gpu

THREADS = 4
ROUNDS = 12


def _run_threads(work, n=THREADS):
    errors = []

    def body(i):
        try:
            work(i)
        except Exception as e:  # noqa: BLE001 -- reported below with the thread index
            errors.append((i, repr(e)))

    ts = [threading.Thread(target=body, args=(i,)) for i in range(n)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=300)
    assert not any(t.is_alive() for t in ts), "a thread did not finish"
    assert not errors, errors


def _cases(seed):
    rng = np.random.default_rng(seed)
    out = []
    for fmt, N, K in (("q4_0", 1000, 4096), ("q8_0", 700, 2048), ("q4_0", 513, 14336)):
        w = rng.standard_normal((N, K)).astype(np.float32)
        wq = (o.quantize_q4_0 if fmt == "q4_0" else o.quantize_q8_0)(w)
        x = rng.standard_normal(K).astype(np.float32)
        out.append((fmt, N, K, x, wq))
    return out


class TestConcurrentCallers:
    def test_quantized_gemv_from_four_threads(self):
        import simd_ml_kernels as sk
        cases = _cases(1)
        expect = [getattr(sk, f"gemv_{fmt}")(x, wq, N, K) for fmt, N, K, x, wq in cases]

        def work(i):
            for r in range(ROUNDS):
                j = (i + r) % len(cases)
                fmt, N, K, x, wq = cases[j]
                y = getattr(sk, f"gemv_{fmt}")(x, wq, N, K)
                np.testing.assert_array_equal(y.view(np.uint32), expect[j].view(np.uint32))

        _run_threads(work)

    def test_read_only_weights_pinned_and_unpinned_while_in_use(self):
        """Read-only weights go device-resident on first use; one thread unpins and re-pins them
        while three others compute with them: no call may read a freed copy."""
        import simd_ml_kernels as sk
        from simd_ml_kernels import _core
        cases = _cases(2)
        for c in cases:
            c[4].setflags(write=False)
        expect = [getattr(sk, f"gemv_{fmt}")(x, wq, N, K) for fmt, N, K, x, wq in cases]
        stop = threading.Event()

        def work(i):
            if i == 0:
                while not stop.is_set():
                    for c in cases:
                        _core._unpin(c[4])
                        _core._pin(c[4])
                return
            try:
                for r in range(ROUNDS):
                    j = (i + r) % len(cases)
                    fmt, N, K, x, wq = cases[j]
                    y = getattr(sk, f"gemv_{fmt}")(x, wq, N, K)
                    np.testing.assert_array_equal(y.view(np.uint32), expect[j].view(np.uint32))
            finally:
                if i == 1:
                    stop.set()

        _run_threads(work)
        for c in cases:
            _core._unpin(c[4])

    def test_fp16_products_and_settings_changes(self):
        """FP16 trans_b products from three threads while a fourth rewrites the (default)
        diagnostics settings: every product keeps its bits."""
        import simd_ml_kernels as sk
        rng = np.random.default_rng(3)
        A = rng.standard_normal((2, 4096)).astype(np.float16)
        W = (rng.standard_normal((3000, 4096)) * 0.02).astype(np.float16)
        expect = sk.sgemm_f16(A, W, trans_b=True)
        stop = threading.Event()

        def work(i):
            if i == 0:
                while not stop.is_set():
                    g.call("smk_set_gemv_tuning", 0, 0, 0, 0)
                    g.call("smk_set_q4_order", 1)
                    g.call("smk_set_q4_mfma_min_rows", 0)
                return
            try:
                for _ in range(ROUNDS):
                    C = sk.sgemm_f16(A, W, trans_b=True)
                    np.testing.assert_array_equal(C.view(np.uint32), expect.view(np.uint32))
            finally:
                if i == 1:
                    stop.set()

        _run_threads(work)

    def test_batched_q4_0_threads_share_the_null_stream(self):
        """Two threads enqueue matrix-core Q4_0 products (which use a scratch buffer) on the same
        stream, the null stream: each thread has its own scratch, so the rows stay exact."""
        rng = np.random.default_rng(4)
        M, N, K = 8, 640, 4096
        jobs = []
        for _ in range(2):
            X = rng.standard_normal((M, K)).astype(np.float32)
            wq = o.quantize_q4_0(rng.standard_normal((N, K)).astype(np.float32))
            ref = np.stack([o.gemv_q4_0_simd(X[m], wq, N, K) for m in range(M)])
            jobs.append((g.dev(X), g.dev(wq), ref))

        def work(i):
            xd, wd, ref = jobs[i % 2]
            for _ in range(ROUNDS):
                yd = g.empty(4 * M * N)
                g.call("smk_d_gemm_q4_0", M, N, K, g.ptr(xd), K, g.ptr(wd), g.ptr(yd), N, None)
                g.call("smk_stream_synchronize", None)
                Y = yd.numpy(np.float32, M * N).reshape(M, N)
                np.testing.assert_array_equal(Y.view(np.uint32), ref.view(np.uint32))

        _run_threads(work)


class TestForcedTuningErrors:
    def test_forced_setting_that_does_not_fit_says_so(self):
        """A forced lanes/threads setting that cannot run a shape fails with a message naming
        the setting (and the default restores the built-in choice)."""
        x = np.random.default_rng(5).standard_normal(14336).astype(np.float32)
        wq = o.quantize_q4_0(np.random.default_rng(6).standard_normal((64, 14336)).astype(np.float32))
        xd, wd, yd = g.dev(x), g.dev(wq), g.empty(4 * 64)
        g.call("smk_set_q4_tiles", -1)
        g.call("smk_set_gemv_tuning", 8, 0, 1024, 0)
        try:
            with pytest.raises(RuntimeError, match="forced tuning"):
                g.call("smk_d_gemv_q4_0", 64, 14336, g.ptr(xd), g.ptr(wd), g.ptr(yd), None)
        finally:
            g.call("smk_set_gemv_tuning", 0, 0, 0, 0)
            g.call("smk_set_q4_tiles", 0)
        g.call("smk_d_gemv_q4_0", 64, 14336, g.ptr(xd), g.ptr(wd), g.ptr(yd), None)
        y = g.host(yd, np.float32, 64)
        np.testing.assert_array_equal(y.view(np.uint32), o.gemv_q4_0_simd(x, wq, 64, 14336).view(np.uint32))
