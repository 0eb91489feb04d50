"""Helpers that read the reference's golden vectors (tests/golden/) and map
fixture file names to the reference's parameter names (name_scope paths)."""
from __future__ import annotations

import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "vision-rs_amd"))
from vrs.synth import seeded_params  # noqa: E402,F401

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(rel: str, shape=None) -> np.ndarray:
    a = np.fromfile(os.path.join(GOLDEN, rel), dtype="<f4")
    return a.reshape(shape) if shape is not None else a


def exists(rel: str) -> bool:
    return os.path.exists(os.path.join(GOLDEN, rel))


_BN = {"w": "weight", "b": "bias", "rm": "running_mean", "rv": "running_var"}


def conv_block_params(family: str, file_prefix: str, name: str, out: dict, cout=None) -> None:
    """<file_prefix>_conv_w.bin / _bn_{w,b,rm,rv}.bin -> <name>.conv.weight, <name>.bn.*"""
    w = load(f"{family}/{file_prefix}_conv_w.bin")
    bnw = load(f"{family}/{file_prefix}_bn_w.bin")
    co = bnw.shape[0]
    out[f"{name}.conv.weight"] = w.reshape(co, -1)  # reshaped to 4-D by the caller
    for k, v in _BN.items():
        out[f"{name}.bn.{v}"] = load(f"{family}/{file_prefix}_bn_{k}.bin")


def fixture_prefix_to_name(p: str) -> str:
    """Fixture prefixes (tests/fixtures/*/generate*.py save_conv_block) -> reference scopes."""
    table = {
        "cv1": "cv1", "cv2": "cv2",
        "m0_cv1": "m.0.cv1", "m0_cv2": "m.0.cv2",
        "m0_icv1": "m.0.cv1", "m0_icv2": "m.0.cv2", "m0_icv3": "m.0.cv3",
        "m0_m0_cv1": "m.0.m.0.cv1", "m0_m0_cv2": "m.0.m.0.cv2",
        "m0_m1_cv1": "m.0.m.1.cv1", "m0_m1_cv2": "m.0.m.1.cv2",
        "m0_attn_qkv": "m.0.attn.qkv", "m0_attn_proj": "m.0.attn.proj", "m0_attn_pe": "m.0.attn.pe",
        "m0_ffn0": "m.0.ffn.0", "m0_ffn1": "m.0.ffn.1",
    }
    return table[p]


def block_params(family: str, shapes: dict) -> dict:
    """Load every conv block of a fixture family.  ``shapes`` maps reference
    param prefix -> conv weight shape (Cout, Cin/g, k, k)."""
    out = {}
    files = sorted(f for f in os.listdir(os.path.join(GOLDEN, family)) if f.endswith("_conv_w.bin"))
    for f in files:
        pre = f[: -len("_conv_w.bin")]
        name = fixture_prefix_to_name(pre)
        conv_block_params(family, pre, name, out)
        out[f"{name}.conv.weight"] = out[f"{name}.conv.weight"].reshape(shapes[name])
    return out


def max_rel_err(got: np.ndarray, ref: np.ndarray, floor: float) -> float:
    """max |got-ref| / max(|ref|, floor) -- elementwise relative with an absolute floor."""
    got = np.asarray(got, np.float64); ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), floor)))
