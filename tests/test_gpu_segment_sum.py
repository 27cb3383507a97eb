"""Per-frame sums (mlcg_segment_sum) against a float64 reference: short and
long segments (a prior's per-interaction energies reach 71,556 values a
frame), empty segments, segment starts at every 16-byte alignment, and a
strided input.  The bound 1e-6 sum|v| is what a compensated sum meets and a
plain float32 sum of the long segments (error up to n u sum|v|) need not."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ref(v, ptr):
    v = v.double().cpu().numpy()
    p = ptr.cpu().numpy()
    s = np.array([v[p[b]:p[b + 1]].sum() for b in range(len(p) - 1)])
    a = np.array([np.abs(v[p[b]:p[b + 1]]).sum() for b in range(len(p) - 1)])
    return s, a


@pytest.mark.parametrize("lengths", [
    [268] * 100,                                   # SchNet energies per frame
    [71556] * 7 + [0, 3, 1, 71555, 5, 0],           # repulsion energies, ragged, empty
    [1, 2, 3, 4, 5, 6, 7, 8, 9, 1025, 4099, 0],    # every start alignment, short runs
])
def test_segment_sum_matches_float64(lengths):
    from mlcg_amd import ops

    torch.manual_seed(3)
    ptr = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int64,
                       device="cuda")
    n = int(ptr[-1])
    v = (torch.randn(n, device="cuda") * 3.0 + 0.5)
    print(f"segments {len(lengths)} values {n}", flush=True)
    got = ops.segment_sum(v, ptr).double().cpu().numpy()
    want, mag = _ref(v, ptr)
    err = np.abs(got - want)
    assert np.all(err <= 1e-6 * mag + 1e-30), float((err / (mag + 1e-30)).max())


def test_segment_sum_strided_through_the_c_abi():
    from mlcg_amd import _lib

    torch.manual_seed(4)
    lengths = [300, 0, 5000, 17]
    ptr = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int64,
                       device="cuda")
    n = int(ptr[-1])
    base = torch.randn(n, 3, device="cuda")
    out = torch.full((len(lengths),), 7.0, device="cuda")
    lib = _lib.load()
    st = lib.mlcg_segment_sum(_lib.ptr(base[:, 1]), 3, _lib.ptr(ptr), len(lengths),
                              _lib.ptr(out), _lib.stream_handle())
    assert st == 0
    torch.cuda.synchronize()
    want, mag = _ref(base[:, 1].contiguous(), ptr)
    err = np.abs(out.double().cpu().numpy() - want)
    assert np.all(err <= 1e-6 * mag + 1e-30)
