"""CPU oracle for the vision-rs YOLO26 inference hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the thing
measured or shipped.  The product (vision-rs_amd/, libvrs.so) never imports it.

This module binds the C restatement in oracle/vrs_oracle.c (built by
oracle/Makefile into oracle/_build/liboracle.so) and exposes NCHW float32
numpy functions.  Each C function cites the reference file:line it follows.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# ORACLE_SO selects another build of the same source (the sanitizer build of
# `make -C oracle sanitize`)
_SO = os.environ.get("ORACLE_SO") or os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        _lib = C.CDLL(_SO)
        f32p = C.POINTER(C.c_float)
        i32p = C.POINTER(C.c_int)
        _lib.orc_conv2d.argtypes = [f32p, C.c_int, C.c_int, C.c_int, C.c_int, f32p, C.c_int, C.c_int,
                                    C.c_int, C.c_int, C.c_int, C.c_int, f32p, f32p]
        _lib.orc_bn_fold.argtypes = [f32p, f32p, f32p, f32p, C.c_float, C.c_int, f32p, f32p]
        _lib.orc_affine_act.argtypes = [f32p, C.c_int, C.c_int, C.c_int, f32p, f32p, C.c_int]
        _lib.orc_bn_train.argtypes = [f32p, C.c_int, C.c_int, C.c_int, f32p, f32p, C.c_float]
        _lib.orc_silu.argtypes = [f32p, f32p, C.c_long]
        _lib.orc_sigmoid.argtypes = [f32p, f32p, C.c_long]
        _lib.orc_maxpool2d.argtypes = [f32p] + [C.c_int] * 7 + [f32p]
        _lib.orc_upsample_nearest.argtypes = [f32p] + [C.c_int] * 6 + [f32p]
        _lib.orc_psa_attention.argtypes = [f32p] + [C.c_int] * 5 + [f32p]
        _lib.orc_detect_decode_grid.argtypes = [f32p, f32p, f32p, f32p, C.c_int, C.c_int, f32p]
        _lib.orc_detect_postprocess.argtypes = [f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int, i32p,
                                                C.c_int, C.c_float, C.c_int, i32p, f32p, i32p, i32p, f32p]
        _lib.orc_detect_unletterbox.argtypes = [C.c_int, C.c_int, C.c_int, i32p, i32p, f32p, f32p]
        _lib.orc_letterbox.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, f32p, f32p, i32p]
        _lib.orc_msda.argtypes = [f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, i32p, i32p,
                                  f32p, f32p, f32p, C.c_int, C.c_int, f32p]
        _lib.orc_add.argtypes = [f32p, f32p, f32p, C.c_long]
        _lib.orc_num_threads.restype = C.c_int
        _lib.orc_build_info.restype = C.c_char_p
    return _lib


def _f(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _i(a):
    return a.ctypes.data_as(C.POINTER(C.c_int))


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def build_info() -> str:
    """Compiler and flags of the oracle library."""
    return lib().orc_build_info().decode()


def num_threads() -> int:
    return int(lib().orc_num_threads())


def conv2d(x, w, stride=1, pad=None, groups=1, bias=None):
    """NCHW conv; pad defaults to k//2 as blocks/conv.rs:36."""
    x = _c32(x); w = _c32(w)
    B, Cin, H, W = x.shape
    Cout, _, kh, kw = w.shape
    if pad is None:
        pad = kh // 2
    Ho = (H + 2 * pad - kh) // stride + 1
    Wo = (W + 2 * pad - kw) // stride + 1
    y = np.empty((B, Cout, Ho, Wo), np.float32)
    b = _c32(bias) if bias is not None else None
    lib().orc_conv2d(_f(x), B, Cin, H, W, _f(w), Cout, kh, kw, stride, pad, groups,
                     _f(b) if b is not None else None, _f(y))
    return y


def bn_fold(gamma, beta, mean, var, eps):
    C_ = gamma.shape[0]
    s = np.empty(C_, np.float32); t = np.empty(C_, np.float32)
    lib().orc_bn_fold(_f(_c32(gamma)), _f(_c32(beta)), _f(_c32(mean)), _f(_c32(var)), eps, C_, _f(s), _f(t))
    return s, t


def affine_act(y, scale, shift, act):
    """In place: y = act(scale*y + shift); act 0 none, 1 SiLU."""
    B, C_, H, W = y.shape
    lib().orc_affine_act(_f(y), B, C_, H * W, _f(_c32(scale)) if scale is not None else None,
                         _f(_c32(shift)) if shift is not None else None, act)
    return y


def bn_train(y, gamma, beta, eps):
    B, C_, H, W = y.shape
    lib().orc_bn_train(_f(y), B, C_, H * W, _f(_c32(gamma)), _f(_c32(beta)), eps)
    return y


def silu(x):
    x = _c32(x); y = np.empty_like(x)
    lib().orc_silu(_f(x), _f(y), x.size)
    return y


def sigmoid(x):
    x = _c32(x); y = np.empty_like(x)
    lib().orc_sigmoid(_f(x), _f(y), x.size)
    return y


def maxpool2d(x, k=5, s=1, p=2):
    x = _c32(x)
    B, C_, H, W = x.shape
    Ho = (H + 2 * p - k) // s + 1; Wo = (W + 2 * p - k) // s + 1
    y = np.empty((B, C_, Ho, Wo), np.float32)
    lib().orc_maxpool2d(_f(x), B, C_, H, W, k, s, p, _f(y))
    return y


def upsample_nearest(x, sh=2, sw=2):
    x = _c32(x)
    B, C_, H, W = x.shape
    y = np.empty((B, C_, H * sh, W * sw), np.float32)
    lib().orc_upsample_nearest(_f(x), B, C_, H, W, sh, sw, _f(y))
    return y


def psa_attention(qkv, heads, kd, vd):
    """qkv [B, heads*(2kd+vd), H, W] -> attention output [B, heads*vd, H, W]."""
    qkv = _c32(qkv)
    B, Cq, H, W = qkv.shape
    assert Cq == heads * (2 * kd + vd)
    out = np.empty((B, heads * vd, H, W), np.float32)
    lib().orc_psa_attention(_f(qkv), B, heads, kd, vd, H * W, _f(out))
    return out


def detect_decode_grid(boxes, ax, ay, strides):
    boxes = _c32(boxes)
    B = boxes.shape[0]; A = ax.shape[0]
    out = np.empty_like(boxes)
    lib().orc_detect_decode_grid(_f(boxes), _f(_c32(ax)), _f(_c32(ay)), _f(_c32(strides)), B, A, _f(out))
    return out


def detect_postprocess(boxes, scores, nc, img_h, img_w, strides=(8, 16, 32), thr=0.25, max_det=300):
    boxes = _c32(boxes); scores = _c32(scores)
    B = boxes.shape[0]
    st = np.ascontiguousarray(strides, dtype=np.int32)
    count = np.zeros(B, np.int32)
    sc = np.zeros((B, max_det), np.float32)
    cl = np.zeros((B, max_det), np.int32)
    an = np.zeros((B, max_det), np.int32)
    xy = np.zeros((B, max_det, 4), np.float32)
    lib().orc_detect_postprocess(_f(boxes), _f(scores), B, nc, img_h, img_w, _i(st), len(strides),
                                 thr, max_det, _i(count), _f(sc), _i(cl), _i(an), _f(xy))
    return count, sc, cl, an, xy


def detect_unletterbox(count, xywh, orig_wh, img_size):
    """xywh [B,max_det,4] letterbox pixels -> normalised original-image boxes
    (examples/yolo26.rs:1531-1547)."""
    xywh = _c32(xywh)
    B, max_det, _ = xywh.shape
    count = np.ascontiguousarray(count, np.int32)
    wh = np.ascontiguousarray(orig_wh, np.int32).reshape(B, 2)
    out = np.empty_like(xywh)
    lib().orc_detect_unletterbox(B, max_det, img_size, _i(wh), _i(count), _f(xywh), _f(out))
    return out


def letterbox(img, img_size, resized=False):
    """RGB8 image [h, w, 3] (uint8) -> model input [3, img_size, img_size]
    float32 (preprocess_image_raw, examples/yolo26.rs:1229-1253).  With
    resized=True also returns the Triangle-resized [new_h, new_w, 3] float32
    values before rounding to u8."""
    img = np.ascontiguousarray(img, np.uint8)
    h, w, _ = img.shape
    out = np.empty((3, img_size, img_size), np.float32)
    nwh = np.zeros(2, np.int32)
    scale = img_size / max(w, h)
    cap = 3 * (int(w * scale + 1)) * (int(h * scale + 1)) + 3
    res = np.empty(cap, np.float32)
    lib().orc_letterbox(img.ctypes.data, w, h, img_size, _f(out), _f(res), _i(nwh))
    if not resized:
        return out
    nw, nh = int(nwh[0]), int(nwh[1])
    return out, res[: 3 * nw * nh].reshape(nh, nw, 3).copy()


def msda(value, shapes, ref, off, attw):
    """value [B,S,heads,Dh]; shapes [(H,W)]*L; ref [B,Q,2]; off [B,Q,heads,L,P,2];
    attw [B,Q,heads,L,P] -> out [B,Q,heads*Dh]."""
    value = _c32(value); ref = _c32(ref); off = _c32(off); attw = _c32(attw)
    B, S, heads, Dh = value.shape
    _, Q, _, L, P, _ = off.shape
    sh = np.ascontiguousarray(np.array(shapes, np.int32).reshape(L, 2))
    starts = np.zeros(L, np.int32)
    starts[1:] = np.cumsum(sh[:, 0] * sh[:, 1])[:-1]
    out = np.empty((B, Q, heads * Dh), np.float32)
    lib().orc_msda(_f(value), B, S, heads, Dh, L, _i(sh), _i(starts), _f(ref), _f(off), _f(attw), Q, P, _f(out))
    return out
