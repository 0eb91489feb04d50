"""Shared helpers for the GPU parity tests (import only from tests marked gpu)."""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "vision-rs_amd")
if PKG not in sys.path:
    sys.path.insert(0, PKG)

import vrs  # noqa: E402

_CTX = None


def ctx():
    global _CTX
    if _CTX is None:
        import torch
        assert torch.cuda.is_available(), "GPU tests need a device"
        torch.cuda.init()
        _CTX = vrs.Context(0)
    return _CTX


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest bfloat16 (ties to even), back as float32."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def rounder(dtype):
    return bf16_round if dtype == vrs.BF16 else (lambda a: np.ascontiguousarray(a, np.float32))


def tdtype(dtype):
    import torch
    return torch.bfloat16 if dtype == vrs.BF16 else torch.float32


def to_nhwc(x_nchw: np.ndarray, dtype, pitch=None, c_off=0):
    """NCHW float32 -> device [n,h,w,pitch] tensor holding x in channels [c_off, c_off+c).

    vrs.nhwc() keeps only the tensor's address: keep the tensor itself alive
    (a named variable) until the kernel reading it has run, or the caching
    allocator may hand its memory to the next allocation first."""
    import torch
    n, c, h, w = x_nchw.shape
    pitch = c if pitch is None else pitch
    t = torch.zeros((n, h, w, pitch), dtype=tdtype(dtype), device="cuda")
    t[..., c_off:c_off + c] = torch.from_numpy(np.ascontiguousarray(x_nchw.transpose(0, 2, 3, 1))).to(
        "cuda", tdtype(dtype))
    return t


def from_nhwc(t, c=None, c_off=0) -> np.ndarray:
    c = t.shape[-1] - c_off if c is None else c
    return t[..., c_off:c_off + c].float().cpu().numpy().transpose(0, 3, 1, 2).copy()


def rel_err(got, ref, floor_frac=1e-2):
    """max |got-ref| / max(|ref|, floor_frac * rms(ref))."""
    got = np.asarray(got, np.float64); ref = np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 1.0
    floor = max(floor_frac * rms, 1e-30)
    return float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), floor))) if ref.size else 0.0


def dev(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to("cuda") if dtype is None else t.to("cuda", dtype)
