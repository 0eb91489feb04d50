"""Graph-structure tests without a GPU (record-only models), mirroring the
reference's tests/test_yolo26n_graph.rs, tests/test_c2psa_yolo26.rs and
tests/test_sppf_yolo26.rs: output shapes, parameter names/shapes, and that the
C++ builders consume exactly the parameters the oracle wiring consumes."""
import numpy as np
import pytest

from gpu_util import vrs
from oracle import yolo26 as Y
from vrs.synth import seeded_params


class Recorder(dict):
    """Params dict that records which names the oracle wiring reads."""

    def __init__(self, P, eps=1e-3):
        super().__init__(P)
        self.eps = eps
        self.act_q = lambda t: t
        self.fp8 = {}
        self.observe = None
        self.store8 = {}
        self.used = set()

    def __getitem__(self, k):
        self.used.add(k)
        return super().__getitem__(k)


def record(desc, h=64, w=64, batch=2):
    return vrs.Model(None, desc, batch, h, w)


def test_yolo26n_output_shapes_64():
    # tests/test_yolo26n_graph.rs:82-96: boxes [2, 336], scores [2, 6720] at 64x64
    m = record(vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant="n", one2one=False))
    assert m.output_shapes() == [(2, 336), (2, 6720)]


def test_yolo26m_640_outputs_and_params():
    m = record(vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant="m"), 640, 640, 64)
    assert m.output_shapes() == [(64, 4 * 8400), (64, 80 * 8400)]
    specs = m.params()
    numel = sum(int(np.prod(s)) for _, s in specs)
    assert 20.0e6 < numel < 20.6e6  # ~20.3 M parameters (YOLO26m)
    convs = [n for n, s in specs if len(s) == 4]
    assert len(convs) == 102  # 94 dense + 8 depthwise
    assert sum(1 for n, s in specs if len(s) == 4 and s[1] == 1 and s[2] == 3) == 8


@pytest.mark.parametrize("variant", ["n", "s", "m", "l", "x"])
@pytest.mark.parametrize("one2one", [True, False])
def test_param_names_match_oracle_wiring(variant, one2one):
    m = record(vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant=variant, one2one=one2one), 64, 64, 1)
    specs = m.params()
    P = Recorder(seeded_params(specs))
    x = np.random.default_rng(0).uniform(0, 1, (1, 3, 64, 64)).astype(np.float32)
    boxes, scores = Y.yolo26(80, variant, one2one)(P, x)
    assert P.used == set(n for n, _ in specs)
    assert boxes.shape == m.output_shapes()[0] and scores.shape == m.output_shapes()[1]


def test_one2one_head_names():
    specs = dict(record(vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant="n", one2one=True)).params())
    assert "model.23.one2one_cv2.0.2.weight" in specs and "model.23.one2one_cv3.2.2.bias" in specs
    assert specs["model.23.one2one_cv3.0.0.0.conv.weight"] == (64, 1, 3, 3)  # DWConv on ch[0]
    assert specs["model.10.m.0.attn.qkv.conv.weight"] == (256, 128, 1, 1)   # 2 heads x (32+32+64)


@pytest.mark.parametrize("desc,ref", [
    (vrs.block(vrs.BLOCK_C3K2, 128, 128, n=1, c3k=True, shortcut=True, e=0.5),
     lambda: Y.c3k2(128, 128, 1, True, True, 0.5)),
    (vrs.block(vrs.BLOCK_C2PSA, 256, 256, n=1, e=0.5), lambda: Y.c2psa(256, 256, 1, 0.5)),
    (vrs.block(vrs.BLOCK_SPPF, 32, 32, shortcut=False), lambda: Y.sppf(32, 32, False)),
    (vrs.block(vrs.BLOCK_C3K2_PSA, 384, 256, n=1, shortcut=True, e=0.5), lambda: Y.c3k2_psa(384, 256, 1, True, 0.5)),
])
def test_block_params_match_oracle(desc, ref):
    m = record(desc, 4, 4)
    P = Recorder(seeded_params(m.params()))
    x = np.zeros((2, desc.c_in, 4, 4), np.float32)
    y = ref()(P, "", x)
    assert P.used == set(n for n, _ in m.params())
    assert m.output_shapes() == [y.shape]


def test_record_only_model_cannot_run():
    m = record(vrs.block(vrs.BLOCK_SPPF, 32, 32))
    with pytest.raises(vrs.VrsError) as e:
        m.load(seeded_params(m.params()))
    assert e.value.code == -7


def test_grouped_conv_block_params():
    # conv_bn with 1 < g < c (blocks/conv.rs:51-69): weight [c_out, c_in/g, k, k];
    # g = c_in = c_out is the depthwise form; g must divide both channel counts
    specs = dict(record(vrs.block(vrs.BLOCK_CONV, 64, 96, k=3, g=4, conv_kind=vrs.CONV_BN), 8, 8).params())
    assert specs["conv.weight"] == (96, 16, 3, 3) and specs["bn.running_var"] == (96,)
    specs = dict(record(vrs.block(vrs.BLOCK_CONV, 64, 64, k=3, g=64, conv_kind=vrs.CONV_BN), 8, 8).params())
    assert specs["conv.weight"] == (64, 1, 3, 3)
    for c_in, c_out, g, kind, code in [(64, 96, 5, vrs.CONV_BN, -2), (64, 64, 2, vrs.CONV_PLAIN, -3)]:
        with pytest.raises(vrs.VrsError) as e:
            record(vrs.block(vrs.BLOCK_CONV, c_in, c_out, k=3, g=g, conv_kind=kind), 8, 8)
        assert e.value.code == code


@pytest.mark.parametrize("one2one", [True, False])
def test_detect_block_params_and_outputs(one2one):
    # detect::<D>(nc, &ch, head) (blocks/detect.rs:108-172) as its own block:
    # the parameters the oracle's detect reads, DetectOutput's shapes
    chs = (64, 128, 256)
    m = record(vrs.block(vrs.BLOCK_DETECT, chs[0], nc=80, one2one=one2one, ch=chs), 16, 16, 2)
    A = 16 * 16 + 8 * 8 + 4 * 4
    assert m.output_shapes() == [(2, 4 * A), (2, 80 * A)]
    P = Recorder(seeded_params(m.params()))
    feats = [np.zeros((2, c, 16 >> i, 16 >> i), np.float32) for i, c in enumerate(chs)]
    boxes, scores = Y.detect(80, list(chs), one2one)(P, "", feats)
    assert P.used == set(n for n, _ in m.params())
    assert boxes.shape == (2, 4 * A) and scores.shape == (2, 80 * A)
    head = "one2one_cv" if one2one else "cv"
    assert dict(m.params())[f"{head}2.0.0.conv.weight"] == (16, 64, 3, 3)   # c2 = max(16, 64/4, 4)


def test_detect_block_rejections():
    for ch, c_in, hw in [((64, 128, 0), 64, 16), ((64, 128, 256), 32, 16), ((64, 128, 256), 64, 18)]:
        with pytest.raises(vrs.VrsError):
            record(vrs.block(vrs.BLOCK_DETECT, c_in, nc=80, ch=ch), hw, hw, 1)
