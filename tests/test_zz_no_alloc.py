"""ta_centroid_accumulate_bf16_noalloc — the allocation-free variant of
ta_centroid_accumulate_bf16 (partial rows in a static device array) — against
the allocating entry point through the C-ABI: the same kernels and order, so
the F64 sums must agree bit for bit, on two calls in a row (the second with a
smaller input, so the static array still holds the first call's larger set
of partial rows), each also within 1e-5 of the oracle's F64 sums.  An input
over the array's capacity is refused before anything is launched."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
import tadapt
from tadapt import call, ptr as P

pytestmark = pytest.mark.gpu

DEV = "cuda"
RNG = np.random.default_rng(97)


def S():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def rbf(*shape, scale=1.0):
    return O.bf16_from_f32((RNG.standard_normal(shape) * scale).astype(np.float32))


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def test_noalloc_matches_allocating_entry_point():
    D = 1536
    for BT in (8192, 1000):  # 512 partial rows, then 63 (the tail block partly filled)
        h, g = rbf(BT, D), rbf(BT, D, scale=1e-3)
        th, tg = dev(h.view(np.int16)), dev(g.view(np.int16))
        init = RNG.standard_normal(D + 1)
        a_ref = torch.from_numpy(init.copy()).to(DEV)
        a_na = torch.from_numpy(init.copy()).to(DEV)
        call("ta_centroid_accumulate_bf16", P(th), P(tg), BT, D, P(a_ref), S())
        call("ta_centroid_accumulate_bf16_noalloc", P(th), P(tg), BT, D, P(a_na), S())
        torch.cuda.synchronize()
        got, want = a_na.cpu().numpy(), a_ref.cpu().numpy()
        assert np.array_equal(got.view(np.uint64), want.view(np.uint64)), BT
        acc, w = O.centroid_accumulate(O.f32_from_bf16(h).reshape(BT, D),
                                       O.f32_from_bf16(g).reshape(BT, D))
        np.testing.assert_allclose(got[:D] - init[:D], acc, rtol=1e-5,
                                   atol=1e-5 * np.abs(acc).max())
        assert abs((got[D] - init[D]) - w) <= 1e-5 * w


def test_noalloc_refuses_inputs_over_its_capacity():
    D = 1536
    BT = 21824 + 16  # one partial row more than the 8 MiB array holds at this D
    t = torch.zeros(1, dtype=torch.int16, device=DEV)
    acc = torch.zeros(D + 1, dtype=torch.float64, device=DEV)
    with pytest.raises(tadapt.BackendError, match="static scratch"):
        call("ta_centroid_accumulate_bf16_noalloc", P(t), P(t), BT, D, P(acc), S())
    assert not torch.any(acc.cpu() != 0)
