"""mlcg_exclusive_scan2_i32_noalloc -- the scan of the radius graph with its
workspace in a device array of the library instead of a caller buffer --
against mlcg_exclusive_scan2_i32, both called through the C ABI: identical
outputs, bit for bit, on two calls in a row (the second with a smaller input,
so stale tile sums of the first call are left in the array), plus the size
limit."""

import pytest
import torch

pytestmark = pytest.mark.gpu

MAX_N = 1 << 24  # MLCG_SCAN_NOALLOC_MAX_N in include/mlcg_hip.h


def _scan_with_workspace(lib, a, b):
    from mlcg_amd import _lib

    n = a.numel()
    out_a = torch.full((n + 1,), -7, dtype=torch.int32, device="cuda")
    out_b = torch.full((n + 1,), -7, dtype=torch.int32, device="cuda")
    ws = torch.full((max(1, int(lib.mlcg_scan_workspace_ints(n))),), -7, dtype=torch.int32,
                    device="cuda")
    st = lib.mlcg_exclusive_scan2_i32(_lib.ptr(a), _lib.ptr(b), n, _lib.ptr(out_a),
                                      _lib.ptr(out_b), _lib.ptr(ws), _lib.stream_handle())
    assert st == 0
    return out_a, out_b


def _scan_noalloc(lib, a, b):
    from mlcg_amd import _lib

    n = a.numel()
    out_a = torch.full((n + 1,), -7, dtype=torch.int32, device="cuda")
    out_b = torch.full((n + 1,), -7, dtype=torch.int32, device="cuda")
    st = lib.mlcg_exclusive_scan2_i32_noalloc(_lib.ptr(a), _lib.ptr(b), n, _lib.ptr(out_a),
                                              _lib.ptr(out_b), _lib.stream_handle())
    assert st == 0
    return out_a, out_b


def test_noalloc_scan_matches_workspace_scan():
    from mlcg_amd import _lib, ops, synthetic

    lib = _lib.load()
    print("noalloc scan: radius-graph degrees of config 3, then a smaller ragged input",
          flush=True)
    b = synthetic.config3(n_frames=512)
    pos = torch.from_numpy(b.pos).cuda()
    batch = torch.from_numpy(b.batch).cuda()
    g = ops.radius_graph(pos, 15.0, batch, False, 1000, with_pairs=True, n_frames=512)
    deg = (g.rowptr[1:] - g.rowptr[:-1]).contiguous()
    udeg = (g.pairptr[1:] - g.pairptr[:-1]).contiguous()
    gen = torch.Generator(device="cuda").manual_seed(7)
    small_a = torch.randint(0, 1000, (5_000,), generator=gen, device="cuda", dtype=torch.int32)
    small_b = torch.randint(0, 3, (5_000,), generator=gen, device="cuda", dtype=torch.int32)
    for a_, b_ in ((deg, udeg), (small_a, small_b)):  # the second call is smaller
        ref = _scan_with_workspace(lib, a_, b_)
        got = _scan_noalloc(lib, a_, b_)
        torch.cuda.synchronize()
        print(f"n={a_.numel()}: totals {int(got[0][-1])}, {int(got[1][-1])}", flush=True)
        assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])
        assert int(got[0][-1]) == int(a_.sum()) and int(got[1][-1]) == int(b_.sum())
    # the degree scan is the CSR of the graph itself
    assert torch.equal(_scan_noalloc(lib, deg, udeg)[0], g.rowptr)
    # an empty input writes the two zero totals
    z = torch.empty(0, dtype=torch.int32, device="cuda")
    za, zb = _scan_noalloc(lib, z, z)
    torch.cuda.synchronize()
    assert za.tolist() == [0] and zb.tolist() == [0]


def test_noalloc_scan_rejects_sizes_past_the_limit():
    from mlcg_amd import _lib

    lib = _lib.load()
    a = torch.zeros(8, dtype=torch.int32, device="cuda")
    out = torch.zeros(9, dtype=torch.int32, device="cuda")
    # rejected on the host, before any launch (the buffers are never touched)
    st = lib.mlcg_exclusive_scan2_i32_noalloc(_lib.ptr(a), _lib.ptr(a), MAX_N + 1, _lib.ptr(out),
                                              _lib.ptr(out), _lib.stream_handle())
    assert _lib.STATUS[st] == "MLCG_ERR_CAPACITY"
    assert _lib.STATUS[lib.mlcg_exclusive_scan2_i32_noalloc(
        _lib.ptr(a), _lib.ptr(a), -1, _lib.ptr(out), _lib.ptr(out),
        _lib.stream_handle())] == "MLCG_ERR_ARGUMENT"
    torch.cuda.synchronize()
    assert int(out.abs().sum()) == 0
