"""The C-ABI library loads, exports every function include/af.h declares, and rejects
invalid arguments before any GPU work (as the reference validates before any CUDA
call: crates/cuda-backend/src/stack.rs:60-84, matvec.rs:198-205,
crates/cuda-backend/src/lib.rs:326-335).  CPU only: no compute call is made."""
import ctypes
import os
import re

import numpy as np
import pytest

from adaforge_amd import _native as N
from adaforge_amd import synth
from adaforge_amd.backend import layer_descs

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "af.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(af_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    lib = N.lib()
    names = declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(N.SIGNATURES), set(names) ^ set(N.SIGNATURES)


def rc_of(fn, *args):
    rc = fn(*args)
    return rc, N.lib().af_last_error().decode()


def test_q4_upload_validation_mirrors_q4matrix_new():
    lib = N.lib()
    out = N.P()
    u8 = lambda a: np.ascontiguousarray(a, np.uint8)
    z18 = u8(np.zeros(18))
    for cols, rows, data in [(31, 1, z18), (32, 0, u8([])), (32, 1, u8(np.zeros(17)))]:
        rc, msg = rc_of(lib.af_q4_upload, data.ctypes.data_as(N.u8p), data.size, cols, rows, ctypes.byref(out))
        assert rc == N.AF_ERR_INVALID, msg
    inf = z18.copy()
    inf[1] = 0x7C
    rc, msg = rc_of(lib.af_q4_upload, inf.ctypes.data_as(N.u8p), 18, 32, 1, ctypes.byref(out))
    assert rc == N.AF_ERR_INVALID and "non-finite" in msg
    big = u8(np.zeros(18 * 513))
    rc, msg = rc_of(lib.af_q4_upload, big.ctypes.data_as(N.u8p), big.size, 32 * 513, 1, ctypes.byref(out))
    assert rc == N.AF_ERR_INVALID and "not supported" in msg


def test_q6_upload_validation_mirrors_q6matrix_new():
    lib = N.lib()
    out = N.P()
    b = np.zeros(210, np.uint8)
    rc, _ = rc_of(lib.af_q6_upload, b.ctypes.data_as(N.u8p), 0, 32, 1, ctypes.byref(out))
    assert rc == N.AF_ERR_INVALID
    b[209] = 0x7C
    rc, _ = rc_of(lib.af_q6_upload, b.ctypes.data_as(N.u8p), 210, 256, 1, ctypes.byref(out))
    assert rc == N.AF_ERR_INVALID


def test_rmsnorm_run_validation_mirrors_rmsnorm_new():
    lib = N.lib()
    w = np.ones(3, np.float32)
    x = np.zeros(3, np.float32)
    y = np.zeros(3, np.float32)
    m = N.f32()
    for eps in (0.0, -1.0, float("nan"), float("inf")):
        rc, msg = rc_of(lib.af_rmsnorm_run, w.ctypes.data_as(N.f32p), 3, eps, x.ctypes.data_as(N.f32p), 1, 0,
                        y.ctypes.data_as(N.f32p), ctypes.byref(m))
        assert rc == N.AF_ERR_INVALID, msg
    bad = np.array([np.nan, 1, 1], np.float32)
    rc, _ = rc_of(lib.af_rmsnorm_run, bad.ctypes.data_as(N.f32p), 3, 1e-6, x.ctypes.data_as(N.f32p), 1, 0,
                  y.ctypes.data_as(N.f32p), ctypes.byref(m))
    assert rc == N.AF_ERR_INVALID
    xi = np.array([np.inf, 0, 0], np.float32)
    rc, _ = rc_of(lib.af_rmsnorm_run, w.ctypes.data_as(N.f32p), 3, 1e-6, xi.ctypes.data_as(N.f32p), 1, 0,
                  y.ctypes.data_as(N.f32p), ctypes.byref(m))
    assert rc == N.AF_ERR_INVALID


def test_matvec_run_rejects_nonfinite_input_before_upload():
    lib = N.lib()
    w = synth.q4("abi", 64, 3)
    x = np.full(64, np.nan, np.float32)
    y = np.zeros(3, np.float32)
    m = N.f32()
    rc, msg = rc_of(lib.af_matvec_run, w.ctypes.data_as(N.u8p), w.size, 64, 3, x.ctypes.data_as(N.f32p), 1, 0,
                    y.ctypes.data_as(N.f32p), ctypes.byref(m))
    assert rc == N.AF_ERR_INVALID and "input" in msg


def _tiny():
    return synth.tiny_model(layers=2, hidden=256, intermediate=512, vocabulary=512, name="abi")


def test_session_open_validation_mirrors_stack_validate():
    lib = N.lib()
    model = _tiny()
    arr, head, keep = layer_descs(model)
    h = N.P()
    rc, msg = rc_of(lib.af_session_open, arr, 2, ctypes.byref(head), 0, ctypes.byref(h))
    assert rc == N.AF_ERR_INVALID, msg
    rc, msg = rc_of(lib.af_session_open, arr, 2, ctypes.byref(head), N.AF_MAX_CONTEXT + 1, ctypes.byref(h))
    assert rc == N.AF_ERR_INVALID
    # a K/V row count that disagrees with the attention config
    arr[1].matrices[1].rows = arr[1].matrices[1].rows - 256
    arr[1].matrices[1].len = arr[1].matrices[1].len - 256 // 32 * 18 * 256
    rc, msg = rc_of(lib.af_session_open, arr, 2, ctypes.byref(head), 16, ctypes.byref(h))
    assert rc == N.AF_ERR_INVALID and "layer 1" in msg
    arr2, head2, keep2 = layer_descs(model)
    head2.cap = 0.0
    rc, msg = rc_of(lib.af_session_open, arr2, 2, ctypes.byref(head2), 16, ctypes.byref(h))
    assert rc == N.AF_ERR_INVALID and "head" in msg
    arr3, head3, keep3 = layer_descs(model)
    arr3[0].attention.q_heads = 3
    rc, msg = rc_of(lib.af_session_open, arr3, 2, ctypes.byref(head3), 16, ctypes.byref(h))
    assert rc == N.AF_ERR_INVALID


def test_generate_rejects_bad_configuration_before_any_gpu_work():
    lib = N.lib()
    model = _tiny()
    arr, head, keep = layer_descs(model)
    p = np.zeros(300, np.uint32)
    s = np.zeros(1, np.uint32)
    o = np.zeros(8, np.uint32)
    n, st, stats = N.sz(), N.i32(), N.GenerationStats()
    args = lambda np_, mn: (arr, 2, ctypes.byref(head), p.ctypes.data_as(N.u32p), np_, s.ctypes.data_as(N.u32p), 1,
                            mn, o.ctypes.data_as(N.u32p), ctypes.byref(n), ctypes.byref(st), ctypes.byref(stats))
    assert lib.af_generate(*args(257, 4)) == N.AF_ERR_INVALID     # prompt > 256 (stack.rs:820-826)
    assert lib.af_generate(*args(4, 0)) == N.AF_ERR_INVALID       # max_new 0
    assert lib.af_generate(*args(4, 129)) == N.AF_ERR_INVALID     # max_new > 128


def test_device_query_reports_no_device_or_gfx950():
    info = N.DeviceInfo()
    rc = N.lib().af_device_query(ctypes.byref(info))
    assert rc in (N.AF_OK, N.AF_ERR_NO_DEVICE)
    if rc == N.AF_OK:
        assert info.arch.decode().startswith("gfx950")
