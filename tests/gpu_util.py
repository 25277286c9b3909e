"""Helpers for the GPU parity tests: numpy <-> device tensors and the
comparison metrics used against the CPU oracle.

BF16 data moves as uint16 bit patterns held in torch.int16 storage; torch
only allocates and copies, every computation runs in libtadapt.so.
"""
import numpy as np
import torch

import tadapt

DEV = "cuda:0"

# Device tensors made by dev()/empty_bf16() stay referenced until the test
# ends (tests/conftest.py clears this after a device sync): a tensor whose
# only reference was a temporary would return its block to torch's caching
# allocator while a kernel still has its pointer.
LIVE = []


def dev(a):
    """numpy -> device tensor with the same bits (uint16 -> int16 storage)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16)).to(DEV)
    else:
        t = torch.from_numpy(a).to(DEV)
    LIVE.append(t)
    return t


def empty_bf16(*shape):
    t = torch.empty(shape, dtype=torch.int16, device=DEV)
    LIVE.append(t)
    return t


def host(t, like=None):
    """device tensor -> numpy (int16 storage comes back as uint16)."""
    torch.cuda.synchronize()
    a = t.detach().cpu().numpy()
    if a.dtype == np.int16:
        return a.view(np.uint16)
    return a


def f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def ulp_diff(a_bits, b_bits):
    """|difference| in BF16 ulps between two bit-pattern arrays (sign-aware)."""
    def ordered(x):
        x = np.asarray(x, np.uint16).astype(np.int32)
        return np.where(x & 0x8000, 0x8000 - x, x)  # monotone map of the float order
    return np.abs(ordered(a_bits) - ordered(b_bits))


def assert_bf16_close(got, want, max_ulp=1, frac_exact=0.99, rl2=1e-2, floor=2.0 ** -12,
                      what=""):
    """BF16 outputs of float math.  Every element within max_ulp BF16 ulps of
    the oracle, except where cancellation made the value tiny: there the bound
    is floor * max|want| absolute.  At least frac_exact bit-identical and
    relative L2 <= rl2 over the tensor."""
    got = np.asarray(got, np.uint16).ravel()
    want = np.asarray(want, np.uint16).ravel()
    if not got.size:
        return
    d = ulp_diff(got, want)
    gf, wf = f32(got).astype(np.float64), f32(want).astype(np.float64)
    small = np.abs(gf - wf) <= floor * np.max(np.abs(wf))
    bad = (d > max_ulp) & ~small
    exact = float((d == 0).mean())
    r = rel_l2(gf, wf)
    assert not bad.any() and exact >= frac_exact and r <= rl2, (
        f"{what}: {int(bad.sum())} elements beyond {max_ulp} ulp (worst {int(d.max())}), "
        f"{exact:.5f} exact, rel-L2 {r:.3e}")


def call(name, *args):
    return tadapt.call(name, *args)


P = tadapt.ptr


def S():
    return tadapt.stream()
