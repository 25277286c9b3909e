"""The C++ host API (include/tensor/**) through its test program
tests/cpp/test_host_api, and the pieces of it that the reference's own host
code pins bit for bit: Dataset batches (src/data/dataset.cpp:56-71) and the
cosine schedule (include/tensor/trainer/cosine_schedule.hpp:18-29), both
compiled from the reference sources into oracle/_ref/ by oracle/build_ref.sh
when the reference tree is present.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import oracle as O
import tadapt

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_host_api")
REF = os.path.join(ROOT, "oracle", "_ref", "libref_host.so")


def _binary():
    if not os.path.exists(BIN):
        subprocess.check_call([os.path.join(ROOT, "tests", "cpp", "build.sh")])
    return BIN


def _ref():
    if not os.path.exists(REF):
        pytest.skip("oracle/_ref not built (the reference tree is absent)")
    L = ctypes.CDLL(REF)
    L.ref_cosine_lr.restype = ctypes.c_float
    L.ref_cosine_lr.argtypes = [ctypes.c_float, ctypes.c_int64, ctypes.c_int64, ctypes.c_float,
                                ctypes.c_int64]
    L.ref_dataset_batches.restype = ctypes.c_int64
    L.ref_dataset_batches.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_void_p, ctypes.c_void_p]
    return L


def _lr_grid():
    for warm in (0, 1, 5, 100):
        for total in (1, 50, 1000):
            for step in range(60):
                if total <= warm:
                    continue
                yield warm, total, step


@pytest.fixture(scope="module")
def cpu_run(tmp_path_factory):
    d = tmp_path_factory.mktemp("host_api")
    r = subprocess.run([_binary(), "cpu", str(d)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    return d


def test_host_api_cpu_checks(cpu_run):
    assert (cpu_run / "batches.bin").exists()


def test_dataset_batches_match_reference_and_oracle(cpu_run):
    got = np.fromfile(cpu_run / "batches.bin", np.int32)
    B, T, NB = 3, 10, 5
    data = cpu_run / "data"
    toks = np.concatenate([np.fromfile(data / "a.bin", np.uint32),
                           np.fromfile(data / "b.bin", np.uint32)])
    pos, want = 0, []
    for _ in range(NB):
        i, t, pos = O.next_batch(toks, pos, B, T)
        want += [i, t]
    np.testing.assert_array_equal(got, np.concatenate(want))
    L = _ref()
    inp = np.empty(NB * B * T, np.int32)
    tgt = np.empty(NB * B * T, np.int32)
    n = L.ref_dataset_batches(str(data).encode(), B, T, NB, inp.ctypes.data, tgt.ctypes.data)
    assert n == toks.size
    ref = np.concatenate([np.concatenate([inp[k * B * T:(k + 1) * B * T],
                                          tgt[k * B * T:(k + 1) * B * T]]) for k in range(NB)])
    np.testing.assert_array_equal(got, ref)


def test_cosine_schedule_bit_exact_vs_reference(cpu_run):
    """The C++ header, the engine's exported schedule and the oracle all
    equal the reference's compiled lr_at bit for bit."""
    got = np.fromfile(cpu_run / "lr.bin", np.float32)
    L = _ref()
    lib = tadapt.lib()
    ref, eng, orc = [], [], []
    for warm, total, step in _lr_grid():
        ref.append(L.ref_cosine_lr(3e-4, warm, total, 0.1, step))
        eng.append(lib.ta_cosine_lr(3e-4, warm, total, 0.1, step))
        orc.append(O.cosine_lr(3e-4, warm, total, 0.1, step))
    ref = np.array(ref, np.float32)
    assert got.size == ref.size
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    np.testing.assert_array_equal(np.array(eng, np.float32).view(np.uint32), ref.view(np.uint32))
    np.testing.assert_array_equal(np.array(orc, np.float32).view(np.uint32), ref.view(np.uint32))


def test_adapter_files_match_independent_readers(cpu_run):
    """The writer's files (src/checkpoint/adapter_writer.cpp:30-150 formats),
    read back with the safetensors library and compared with Python's json:
    adapter.safetensors holds every tensor as flat 1-D BF16 (round to
    nearest even, ties included), its header is the compact JSON with
    sorted keys padded with spaces to a multiple of 8 and the data follow in
    tensor order; optimizer.safetensors holds the exact F32 masters, their
    moments and the F64 centroid sums; adapter.json and train_state.json are
    2-space-indented JSON with sorted keys, byte for byte."""
    import json

    import torch
    from safetensors.torch import load_file

    w = cpu_run / "writer"
    names = [(ln.split()[0], int(ln.split()[1])) for ln in open(w / "names.txt")]
    vals = np.fromfile(w / "values.bin", np.float32)
    sums = np.fromfile(w / "sums.bin", np.float64)
    expect, off = {}, 0
    for n, c in names:
        expect[n] = vals[off:off + c]
        off += c
    assert off == vals.size
    for d in ("ckpt", "final"):
        raw = open(w / d / "adapter.safetensors", "rb").read()
        hl = int.from_bytes(raw[:8], "little")
        hdr, o = {}, 0
        for n, c in names:
            hdr[n] = {"data_offsets": [o, o + 2 * c], "dtype": "BF16", "shape": [c]}
            o += 2 * c
        text = json.dumps(hdr, separators=(",", ":"), sort_keys=True)
        text += " " * (-len(text) % 8)
        assert raw[8:8 + hl].decode() == text and len(raw) == 8 + hl + o
        t = load_file(str(w / d / "adapter.safetensors"))
        assert sorted(t) == sorted(expect)
        for n, c in names:
            want = torch.from_numpy(expect[n].copy()).to(torch.bfloat16)
            assert t[n].dtype == torch.bfloat16 and tuple(t[n].shape) == (c,)
            assert torch.equal(t[n].view(torch.int16), want.view(torch.int16)), n
            # the two ties the C++ side planted: 1 + 2^-8 -> 1, -(1 + 3 * 2^-8) -> -(1 + 2^-6)
            assert t[n][0].item() == 1.0 and t[n][1].item() == -1.015625
    opt = load_file(str(w / "ckpt" / "optimizer.safetensors"))
    assert len(opt) == 3 * len(names) + 1
    for n, c in names:
        assert torch.equal(opt[n], torch.from_numpy(expect[n].copy()))
        for m in (".exp_avg", ".exp_avg_sq"):
            assert opt[n + m].dtype == torch.float32 and tuple(opt[n + m].shape) == (c,)
    assert opt["centroid.sums"].dtype == torch.float64
    np.testing.assert_array_equal(opt["centroid.sums"].numpy(), sums)
    meta = dict(domain='golang/gin "x"', architecture="qwen2", base_model="unknown",
                base_sha="abc123", rank=4, alpha=float(np.float32(0.1)), target_begin=0,
                target_end=1, inject_q=True, inject_k=False, inject_v=True, inject_o=True,
                inject_up=False, inject_down=True, tokens_trained=3584, centroid_dim=16,
                centroid_count=16, step=7, tensor_adapt_version="0.1.0")
    assert open(w / "ckpt" / "adapter.json").read() == json.dumps(meta, indent=2, sort_keys=True)
    meta.update(domain="golang/gin", step=9, tokens_trained=4608)
    assert open(w / "final" / "adapter.json").read() == json.dumps(meta, indent=2, sort_keys=True)
    assert open(w / "ckpt" / "train_state.json").read() == json.dumps(
        {"step": 7, "tokens_consumed": 3584}, indent=2)


@pytest.mark.gpu
def test_host_api_gpu(tmp_path):
    print("case: test_host_api gpu", flush=True)
    r = subprocess.run([_binary(), "gpu", str(tmp_path)], capture_output=True, text=True,
                       timeout=110)
    assert r.returncode == 0, r.stdout + r.stderr[-2000:]


@pytest.mark.gpu
def test_c2_schedule_through_trainer(tmp_path):
    """BASELINE configs[1] on its own schedule through AdaptTrainer: 20 AdamW
    steps of the Qwen2-0.5B shape (B=4 x T=512, r=16 on q,k,v,o) with a
    centroid snapshot every 10 steps; the two snapshot files' layout and
    cumulative C / W, the lr schedule and the merged file are checked in
    tests/cpp/test_host_api.cpp (c2_schedule_tests).  The centroid sums
    themselves are compared with the oracle over c2's first two steps in
    tests/test_gpu_c2.py."""
    print("case: test_host_api c2sched", flush=True)
    r = subprocess.run([_binary(), "c2sched", str(tmp_path)], capture_output=True, text=True,
                       timeout=170)
    assert r.returncode == 0, r.stdout + r.stderr[-2000:]


@pytest.mark.gpu
def test_per_op_classes_match_engine(tmp_path):
    """The per-op classes of include/tensor (Qwen2Base forward/backward,
    AdapterModel, AdamW) composed into the reference trainer's step
    (adapt_trainer.cu:189-253) agree with the step engine over two steps on
    the same base and batches: loss, every gA/gB and the updated masters
    (tests/cpp/test_host_api.cpp perop_tests)."""
    print("case: test_host_api perop", flush=True)
    r = subprocess.run([_binary(), "perop", str(tmp_path)], capture_output=True, text=True,
                       timeout=110)
    print(r.stdout[-3000:])
    assert r.returncode == 0, r.stdout + r.stderr[-2000:]

