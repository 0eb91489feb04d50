"""CPU-side checks of the C ABI: the library loads, exports every symbol
include/vrs.h declares, the Python binding covers them, and host-forced
failures come back as status codes (no kernel is launched here)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from gpu_util import ROOT, vrs

HEADER = os.path.join(ROOT, "include", "vrs.h")


def declared_symbols():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(vrs_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    L = vrs.lib()
    syms = declared_symbols()
    assert len(syms) >= 25
    for s in syms:
        assert hasattr(L, s), s
    assert set(syms) == set(vrs.SIGNATURES), set(syms) ^ set(vrs.SIGNATURES)


def test_code_objects_built_for_gfx950():
    objs = [f for f in os.listdir(vrs.LIB_DIR) if f.endswith(".hsaco")]
    assert {"conv.hsaco", "misc.hsaco", "attn.hsaco", "detect.hsaco", "msda.hsaco"} <= set(objs)
    for f in objs:
        head = open(os.path.join(vrs.LIB_DIR, f), "rb").read(4096)
        # clang offload bundle (hipcc --genco) holding a gfx950 code object
        assert head.startswith(b"__CLANG_OFFLOAD_BUNDLE__") and b"gfx950" in head


def test_missing_code_objects_is_an_error():
    h = C.c_void_p()
    rc = vrs.lib().vrs_ctx_create(0, b"/nonexistent/dir", C.byref(h))
    assert rc == -4 and not h
    assert b"not found" in vrs.lib().vrs_last_error()


def test_null_arguments_rejected_before_any_hip_call():
    L = vrs.lib()
    assert L.vrs_conv2d(None, None, None, None, None, None, None, None, None) == -1
    assert L.vrs_model_forward(None, None, None, None) == -1
    assert L.vrs_msda(None, None, None, None, None, None, None, None) == -1
    d = vrs.DetectDesc(1, 80, 640, 640, 3, (C.c_int32 * 4)(8, 16, 32, 0), 0.25, 5000)
    assert L.vrs_detect_workspace_size(C.byref(d)) == 0  # max_det > 1024 rejected


def test_pack_conv_weight_layout():
    w = np.arange(2 * 3 * 3 * 3, dtype=np.float32).reshape(2, 3, 3, 3)
    out = vrs.pack_conv_weight(w, 1, 8, vrs.F32).view(np.float32).reshape(2, 3, 3, 8)
    assert np.array_equal(out[..., :3], w.transpose(0, 2, 3, 1))
    assert np.all(out[..., 3:] == 0)
    b = vrs.pack_conv_weight(np.array([[[[1.0, 1.00390625, 1.01171875]]]], np.float32).reshape(1, 3, 1, 1), 1, 8,
                             vrs.BF16).view(np.uint16)
    # round to nearest even: 1.00390625 is halfway between 1.0 and 1.0078125 -> 1.0
    assert b[0] == 0x3F80 and b[1] == 0x3F80 and b[2] == 0x3F82
    # depthwise: [C][1][3][3] -> tap-major [9][C]
    dw = np.arange(4 * 9, dtype=np.float32).reshape(4, 1, 3, 3)
    out = vrs.pack_conv_weight(dw, 4, 1, vrs.F32).view(np.float32).reshape(9, 4)
    assert np.array_equal(out, dw.reshape(4, 9).T)


def test_bn_fold_matches_reference_formula():
    g = np.array([2.0, 1.0], np.float32); be = np.array([0.5, 0.0], np.float32)
    mu = np.array([3.0, 0.0], np.float32); var = np.array([3.999, 1.0], np.float32)
    s, t = vrs.bn_fold(g, be, mu, var, 1e-3)
    assert abs(s[0] - 1.0) < 1e-6 and abs(t[0] + 2.5) < 1e-6
    assert s[1] == np.float32(1.0) / np.sqrt(np.float32(1.001))


def test_no_gpu_context_fails_cleanly():
    torch = pytest.importorskip("torch")
    if torch.cuda.device_count() > 0:
        pytest.skip("GPU present")
    h = C.c_void_p()
    rc = vrs.lib().vrs_ctx_create(0, vrs.LIB_DIR.encode(), C.byref(h))
    assert rc in (-1, -5) and not h


def test_pack_conv_weight_fp8_matches_torch():
    """Host e4m3 packing: per-channel step max|w|/448, ties to even, zero pad."""
    import torch
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((6, 5, 3, 3)) * np.exp(rng.uniform(-8, 3, (6, 5, 3, 3)))).astype(np.float32)
    w[0].flat[:8] = [448, -448, 2 ** -9, 2 ** -10, 3 * 2 ** -10, 1.0625, 1.1875, 232]   # step 1.0 on row 0
    q, sc = vrs.pack_conv_weight_fp8(w, cin_pad=8)
    amax = np.abs(w.reshape(6, -1)).max(1)
    assert np.array_equal(sc, (amax / np.float32(448)).astype(np.float32))
    ref = torch.from_numpy(w / sc[:, None, None, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    got = q.reshape(6, 3, 3, 8)
    assert np.array_equal(got[..., :5].transpose(0, 3, 1, 2), ref.numpy())
    assert np.all(got[..., 5:] == 0)

