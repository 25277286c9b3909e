"""The Centroid Accumulator + Merge stress configuration at full size:
4M = 4 * 2^20 token hidden states of dimension 512 (F32) from a seeded
mixture of 16 isotropic Gaussians (means ~ N(0, 1), sigma 0.3), per-token
gradient norms lognormal(0, 1), C += h * n accumulated through the C-ABI
into 64 cumulative snapshots (one every 65536 tokens; snapshot = C / W as
CentroidAccumulator::write_snapshot makes it,
src/centroid/centroid_accumulator.cpp:72-91), then k-means with k = 32,
25 Lloyd iterations, k-means++ seeding, clusters ranked by the total
snapshot weight of their members.

Checks: every snapshot's sums against the oracle's F64 accumulation to
1e-5 relative (the F32 centroid bar) and W to 1e-6; the k-means seeds,
assignments and centers bit-exact against the oracle on the same
snapshots, masses to 1e-12, and masses in descending order.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import DEV, P, S, call, host

pytestmark = pytest.mark.gpu

N_TOK, D, CHUNK, COMPS, K, ITERS = 4 << 20, 512, 65536, 16, 32, 25


def mixture_chunks(seed):
    """The c5 token stream, 65536 tokens at a time: (h [CHUNK, D] F32, n [CHUNK] F32)."""
    r = np.random.default_rng(seed)
    means = r.standard_normal((COMPS, D), dtype=np.float32)
    for _ in range(N_TOK // CHUNK):
        lab = r.integers(0, COMPS, CHUNK)
        h = means[lab] + np.float32(0.3) * r.standard_normal((CHUNK, D), dtype=np.float32)
        n = r.lognormal(0.0, 1.0, CHUNK).astype(np.float32)
        yield h, n


def test_c5_accumulate_and_merge():
    acc = torch.zeros(D + 1, dtype=torch.float64, device=DEV)
    ref, ref_w = np.zeros(D, np.float64), 0.0
    snaps, weights = [], []
    for i, (h, n) in enumerate(mixture_chunks(2026)):
        th, tn = torch.from_numpy(h).to(DEV), torch.from_numpy(n).to(DEV)
        call("ta_centroid_accumulate_f32n", P(th), P(tn), CHUNK, D, P(acc), S())
        ref, ref_w = O.centroid_accumulate_n(h, n, ref, ref_w)
        a = host(acc)
        assert np.max(np.abs(a[:D] - ref)) <= 1e-5 * np.max(np.abs(ref)), i
        assert abs(a[D] - ref_w) <= 1e-6 * ref_w, i
        snaps.append((a[:D] / a[D]).astype(np.float32))
        weights.append(np.float32(a[D]))
    print(f"64 snapshots, W = {weights[-1]:.6e}", flush=True)
    X = np.ascontiguousarray(np.stack(snaps))
    Wt = np.asarray(weights, np.float32)
    C = torch.empty(K * D, dtype=torch.float32, device=DEV)
    A = torch.empty(len(snaps), dtype=torch.int32, device=DEV)
    M = torch.empty(K, dtype=torch.float64, device=DEV)
    Sd = torch.empty(K, dtype=torch.int32, device=DEV)
    tX, tW = torch.from_numpy(X).to(DEV), torch.from_numpy(Wt).to(DEV)
    call("ta_kmeans_pp", P(tX), P(tW), len(snaps), D, K, ITERS, ctypes.c_uint64(5), P(C), P(A),
         P(M), P(Sd), S())
    rc, ra, rm, rs = O.kmeans_pp(X, Wt, K, ITERS, 5)
    assert np.array_equal(host(Sd), rs)
    assert np.array_equal(host(A), ra)
    assert np.array_equal(host(C).reshape(K, D), rc)
    m = host(M)
    assert np.allclose(m, rm, rtol=1e-12)
    assert np.all(np.diff(m) <= 0)
