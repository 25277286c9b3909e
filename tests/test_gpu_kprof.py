"""The kernel timer of the C-ABI (ta_kprof_select / ta_kprof_pause /
ta_kprof_read), which bench.py uses for its roofline line: every unpaused
launch of the selected kernel is timed once, paused launches are not, and
timed calls on several threads (each on its own stream) each take an event
pair of their own."""
import ctypes
import threading

import numpy as np
import pytest
import torch

import oracle as O
import tadapt
from gpu_util import P, S, call, dev, empty_bf16, host

pytestmark = pytest.mark.gpu

M = N = K = 1024  # k_gemm_mid<64> tiles: kernel id 0 (gemm_big)


def test_kprof_counts_timed_launches_across_threads():
    rng = np.random.default_rng(5)
    X = dev(O.bf16_from_f32(rng.standard_normal((M, K)).astype(np.float32)))
    Y = dev(O.bf16_from_f32(rng.standard_normal((N, K)).astype(np.float32) * 0.02))

    def gemm(stream, C):
        call("ta_gemm_rm", 1, 1, M, N, K, ctypes.c_float(1.0), P(X), K, P(Y), K,
             ctypes.c_float(0.0), P(C), N, None, stream)

    C0 = empty_bf16(M, N)
    gemm(S(), C0)
    torch.cuda.synchronize()
    tadapt.kprof_select(0)
    try:
        for i in range(6):
            tadapt.kprof_pause(i % 2 == 1)
            gemm(S(), C0)
        tadapt.kprof_pause(False)
        r = tadapt.kprof_read()
        assert r["launches"] == 3 and r["ms"] > 0
        assert r["flops"] == pytest.approx(3 * 2.0 * M * N * K, rel=1e-9)
        assert "k_gemm" in tadapt.kprof_name(0)

        streams = [torch.cuda.Stream() for _ in range(2)]
        outs = [empty_bf16(M, N) for _ in range(2)]
        errors = []

        def worker(t):
            try:
                for _ in range(5):
                    gemm(ctypes.c_void_p(streams[t].cuda_stream), outs[t])
            except Exception as e:  # reported by the main thread
                errors.append(e)

        threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
        for th in threads:
            th.start()
        for th in threads:
            th.join()
        torch.cuda.synchronize()
        assert not errors, errors
        r = tadapt.kprof_read()
        assert r["launches"] == 10 and r["ms"] > 0
        assert r["flops"] == pytest.approx(10 * 2.0 * M * N * K, rel=1e-9)
        ref = host(C0)
        for t in range(2):
            assert np.array_equal(host(outs[t]), ref)
    finally:
        tadapt.kprof_select(-1)
