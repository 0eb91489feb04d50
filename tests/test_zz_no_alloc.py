"""vrs_detect_postprocess_noalloc (the allocation-free entry point) against
vrs_detect_postprocess with a caller workspace, through the C ABI, on two
calls in a row (the second smaller, reusing the fixed workspace that still
holds the first call's contents), plus its size limit."""
import numpy as np
import pytest

from gpu_util import ctx, dev, vrs

pytestmark = pytest.mark.gpu


def _outs(n, max_det):
    import torch
    return (torch.full((n,), -7, dtype=torch.int32, device="cuda"),
            torch.full((n, max_det), -7.0, device="cuda"),
            torch.full((n, max_det), -7, dtype=torch.int32, device="cuda"),
            torch.full((n, max_det), -7, dtype=torch.int32, device="cuda"),
            torch.full((n, max_det, 4), -7.0, device="cuda"))


def _inputs(n, img, nc, seed):
    rng = np.random.default_rng(seed)
    A = sum((img // s) ** 2 for s in (8, 16, 32))
    boxes = rng.uniform(0, 5, (n, 4 * A)).astype(np.float32)
    scores = rng.normal(-2.5, 2, (n, nc * A)).astype(np.float32)
    scores[0, : nc * 6] = 3.0   # exact ties across classes and anchors
    return dev(boxes), dev(scores)


@pytest.mark.parametrize("calls", [[(64, 640, 80, 0.25, 300), (3, 320, 80, 0.25, 100)],
                                   [(8, 640, 80, 0.001, 1024), (2, 96, 5, 0.3, 7)]])
def test_noalloc_matches_workspace_entry_point(calls):
    import torch
    for i, (n, img, nc, thr, max_det) in enumerate(calls):
        boxes, scores = _inputs(n, img, nc, 100 + i)
        ref = ctx().detect_postprocess(boxes, scores, nc, img, img, (8, 16, 32), thr, max_det)
        got = ctx().detect_postprocess_noalloc(boxes, scores, nc, img, img, _outs(n, max_det), (8, 16, 32), thr)
        torch.cuda.synchronize()
        for a, b in zip(got, ref):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32)), (i, n, img)
        assert int(ref[0].sum()) > 0


def test_noalloc_rejects_sizes_beyond_the_fixed_workspace():
    import torch
    n, img, nc = 72, 640, 80    # 72 * 8400 anchors * 28 bytes > 16 MiB (64 images fit)
    boxes = torch.zeros(n, 4 * 8400, device="cuda")
    scores = torch.zeros(n, nc * 8400, device="cuda")
    with pytest.raises(vrs.VrsError) as e:
        ctx().detect_postprocess_noalloc(boxes, scores, nc, img, img, _outs(n, 10))
    assert e.value.code == -3 and "fixed" in str(e.value)
