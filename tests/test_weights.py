"""Weight ingestion from local .safetensors files (load_weights_from_safetensors,
examples/yolo26.rs:3403-3550), on record-only models (no GPU): key lookup,
the reference's "X.weight" / "X.conv.weight" fallback, dtype conversion,
missing-key accounting and malformed-file errors.  The GPU test in
test_gpu_blocks.py checks that a model loaded from a file computes exactly
what the same model loaded tensor by tensor computes."""
import json
import struct

import numpy as np
import pytest

from gpu_util import vrs
from vrs.synth import seeded_params


def _model():
    return vrs.Model(None, vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant="n"), 1, 64, 64)


def _write(path, tensors):
    """Minimal safetensors writer (independent of the reader under test):
    {name: (dtype string, numpy array)} -> file."""
    header, blobs, off = {}, [], 0
    for name, (dt, a) in tensors.items():
        raw = np.ascontiguousarray(a).tobytes()
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    header["__metadata__"] = {"format": "pt", "note": 'esc " quote \u00e9 /'}   # escapes in the header
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + b"".join(blobs))


def test_load_all_and_count_missing(tmp_path):
    m = _model()
    P = seeded_params(m.params())
    _write(tmp_path / "w.safetensors", {k: ("F32", v) for k, v in P.items()})
    assert m.load_safetensors(tmp_path / "w.safetensors", finalize=False) == (len(P), 0)
    drop = sorted(P)[:3]
    _write(tmp_path / "d.safetensors", {k: ("F32", v) for k, v in P.items() if k not in drop})
    assert _model().load_safetensors(tmp_path / "d.safetensors", finalize=False) == (len(P) - 3, 3)


def test_conv_weight_fallback_both_ways(tmp_path):
    m = _model()
    P = seeded_params(m.params())
    conv = next(k for k in P if k.endswith(".conv.weight"))
    plain = next(k for k in P if k.endswith(".weight") and not k.endswith("conv.weight") and P[k].ndim == 4)
    T = {k: ("F32", v) for k, v in P.items() if k not in (conv, plain)}
    T[conv[: -len(".conv.weight")] + ".weight"] = ("F32", P[conv])              # fused-node naming
    T[plain[: -len(".weight")] + ".conv.weight"] = ("F32", P[plain])            # checkpoint naming
    _write(tmp_path / "w.safetensors", T)
    assert m.load_safetensors(tmp_path / "w.safetensors", finalize=False) == (len(P), 0)


def test_half_bfloat16_double(tmp_path):
    import torch
    from safetensors.torch import save_file
    m = _model()
    P = seeded_params(m.params())
    names = sorted(P)
    T = {}
    for i, k in enumerate(names):
        t = torch.from_numpy(P[k])
        T[k] = t.to([torch.float32, torch.float16, torch.bfloat16, torch.float64][i % 4])
    save_file(T, str(tmp_path / "w.safetensors"))
    assert m.load_safetensors(tmp_path / "w.safetensors", finalize=False) == (len(P), 0)


def test_errors(tmp_path):
    m = _model()
    P = seeded_params(m.params())
    k0 = sorted(P)[0]
    # element count differs from the parameter
    bad = {k: ("F32", v) for k, v in P.items()}
    bad[k0] = ("F32", np.zeros(P[k0].size + 1, np.float32))
    _write(tmp_path / "n.safetensors", bad)
    with pytest.raises(vrs.VrsError) as e:
        _model().load_safetensors(tmp_path / "n.safetensors", finalize=False)
    assert e.value.code == -2
    # integer tensor where a float parameter is expected
    bad[k0] = ("I32", np.zeros(P[k0].shape, np.int32))
    _write(tmp_path / "i.safetensors", bad)
    with pytest.raises(vrs.VrsError) as e:
        _model().load_safetensors(tmp_path / "i.safetensors", finalize=False)
    assert e.value.code == -3
    # truncated data, header length past the end, not JSON, missing file
    _write(tmp_path / "w.safetensors", {k: ("F32", v) for k, v in P.items()})
    raw = (tmp_path / "w.safetensors").read_bytes()
    (tmp_path / "t.safetensors").write_bytes(raw[:-5])
    (tmp_path / "h.safetensors").write_bytes(struct.pack("<Q", len(raw)) + raw[8:])
    (tmp_path / "j.safetensors").write_bytes(struct.pack("<Q", 4) + b"[1,]")
    # a shape whose element count overflows 64 bits (2^96 elements) must be
    # rejected before any size arithmetic, whatever its byte span claims
    hdr = b'{"%s":{"dtype":"F32","shape":[4294967296,4294967296,4294967296],"data_offsets":[0,4]}}' % k0.encode()
    (tmp_path / "o.safetensors").write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 4)
    with pytest.raises(vrs.VrsError) as e:
        _model().load_safetensors(tmp_path / "o.safetensors", finalize=False)
    assert e.value.code == -2 and "overflow" in str(e.value)
    for f in ("t", "h", "j"):
        with pytest.raises(vrs.VrsError):
            _model().load_safetensors(tmp_path / f"{f}.safetensors", finalize=False)
    with pytest.raises(vrs.VrsError):
        _model().load_safetensors(tmp_path / "absent.safetensors", finalize=False)


def test_corrupted_files_fail_cleanly(tmp_path):
    """Random byte and length corruptions of a valid file either load or
    raise VrsError (no crash, no hang)."""
    m0 = _model()
    P = seeded_params(m0.params())
    small = dict(sorted(P.items())[:6])
    _write(tmp_path / "w.safetensors", {k: ("F32", v) for k, v in small.items()})
    raw = bytearray((tmp_path / "w.safetensors").read_bytes())
    hlen = struct.unpack("<Q", raw[:8])[0]
    rng = np.random.default_rng(0)
    outcomes = {"ok": 0, "err": 0}
    for trial in range(300):
        b = bytearray(raw)
        kind = trial % 3
        if kind == 0:      # flip bytes inside the JSON header
            for _ in range(int(rng.integers(1, 4))):
                b[8 + int(rng.integers(0, hlen))] = int(rng.integers(0, 256))
        elif kind == 1:    # truncate anywhere
            b = b[: int(rng.integers(0, len(b)))]
        else:              # corrupt the header length
            b[:8] = struct.pack("<Q", int(rng.integers(0, 2 * len(raw))))
        f = tmp_path / f"c{trial}.safetensors"
        f.write_bytes(bytes(b))
        try:
            _model().load_safetensors(f, finalize=False)
            outcomes["ok"] += 1
        except vrs.VrsError:
            outcomes["err"] += 1
    assert outcomes["err"] > 100
