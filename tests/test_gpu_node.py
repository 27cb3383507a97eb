"""Node-level weight-gradient reduction (mlcg_node_tmm) against fp64 torch
products at ragged row counts, and the node_linear helper's epilogues.

Every element is held to rtol of the tensor's largest element (check with
atol_frac=1.0): node_linear's products run on the fp16 MFMA with split
operands (about 22 significant bits) and node_tmm's on the bf16 MFMA with
three-way splits (each product within 2^-23 of exact, summed in fp32), so an
element's error scales with the terms it sums, not with the element."""

import pytest
import torch

from tests.helpers import check

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("transpose", [False, True])
def test_node_linear_helper(transpose):
    from mlcg_amd import ops

    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn(1000, 128, device="cuda", generator=g)
    W = torch.randn(128, 128, device="cuda", generator=g) / 11
    b = torch.randn(128, device="cuda", generator=g)
    r = torch.randn(1000, 128, device="cuda", generator=g)
    Wd = W.double()
    ref = x.double().mm(Wd if transpose else Wd.t())
    check(ops.node_linear(x, W, transpose=transpose), ref, 1e-6, 'ops.node_linear(x, W, transpose=transpos', atol_frac=1.0)
    out = ops.node_linear(x, W, bias=b, residual=r, transpose=transpose)
    check(out, ref + b.double() + r.double(), 1e-6, 'out', atol_frac=1.0)


@pytest.mark.parametrize("rows", [0, 1, 15, 16, 17, 127, 128, 129, 4095, 4097, 5000, 17920,
                                  128000])
def test_node_tmm(rows):
    from mlcg_amd import ops

    g = torch.Generator(device="cuda").manual_seed(rows + 1)
    a1, b1, a2, b2 = (torch.randn(rows, 128, device="cuda", generator=g) for _ in range(4))
    ref = a1.double().t().mm(b1.double())
    got = ops.node_tmm(a1, b1)
    if rows == 0:
        assert float(got.abs().max()) == 0.0
        return
    check(got, ref, 1e-6, 'got', atol_frac=1.0)
    ref2 = ref + a2.double().t().mm(b2.double())
    check(ops.node_tmm(a1, b1, a2, b2), ref2, 1e-6, 'ops.node_tmm(a1, b1, a2, b2)', atol_frac=1.0)
    # deterministic: bitwise identical on a second call
    assert torch.equal(ops.node_tmm(a1, b1, a2, b2), ops.node_tmm(a1, b1, a2, b2))
    # fused column sums of a1 (bias gradients)
    got, cs = ops.node_tmm(a1, b1, a2, b2, colsum=True)
    check(got, ref2, 1e-6, 'got', atol_frac=1.0)
    check(cs, a1.double().sum(0), 1e-6, 'cs', atol_frac=1.0)
    got, cs = ops.node_tmm(a1, b1, colsum=True)
    check(cs, a1.double().sum(0), 1e-6, 'cs', atol_frac=1.0)


@pytest.mark.parametrize("rows", [0, 1, 33, 1000, 17920, 128000])
@pytest.mark.parametrize("count", [1, 3, 4])
def test_node_tmm_batch(rows, count):
    """Batched weight-gradient reductions (one launch pair for `count`
    problems, with and without the second product and column sums) against
    fp64 products, and run-to-run identical."""
    from mlcg_amd import ops

    print(f"node_tmm_batch rows={rows} count={count}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(7 * rows + count)
    probs, refs = [], []
    for k in range(count):
        a1, b1, a2, b2 = (torch.randn(rows, 128, device="cuda", generator=g) * (10.0 ** k)
                          for _ in range(4))
        two, cs = k % 2 == 0, k != 2
        probs.append((a1, b1, a2 if two else None, b2 if two else None, cs))
        r = a1.double().t().mm(b1.double())
        if two:
            r = r + a2.double().t().mm(b2.double())
        refs.append((r, a1.double().sum(0) if cs else None))
    got = ops.node_tmm_batch(probs, rows, torch.device("cuda"))
    again = ops.node_tmm_batch(probs, rows, torch.device("cuda"))
    for k, (pr, (r, rc)) in enumerate(zip(probs, refs)):
        out, cs = got[k] if pr[4] else (got[k], None)
        out2, cs2 = again[k] if pr[4] else (again[k], None)
        assert torch.equal(out, out2)
        if rows == 0:
            assert float(out.abs().max()) == 0.0
            continue
        check(out, r, 1e-6, f"batch[{k}]", atol_frac=1.0)
        if rc is not None:
            assert torch.equal(cs, cs2)
            check(cs, rc, 1e-6, f"colsum[{k}]", atol_frac=1.0)


def _act64(z, act):
    if act == 0:
        return torch.tanh(z)
    return torch.nn.functional.softplus(z) - torch.log(torch.tensor(2.0, dtype=z.dtype))


def _derivs64(z, act):
    if act == 0:
        s = torch.tanh(z)
        d1 = 1 - s * s
        return d1, -2 * s * d1
    sg = torch.sigmoid(z)
    return sg, sg * (1 - sg)


@pytest.mark.parametrize("rows", [1, 15, 16, 17, 1000, 17920])
@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("act", [0, 1])
def test_node_gemm_epilogues(rows, transpose, act):
    """Every epilogue of mlcg_node_gemm against fp64 torch at ragged row
    counts (tiles of 16 rows) and both weight orientations."""
    from mlcg_amd import ops

    print(f"node_gemm rows={rows} transpose={transpose} act={act}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows * 4 + 2 * int(transpose) + act)
    rnd = lambda *s: torch.randn(*s, device="cuda", generator=g)  # noqa: E731
    x, r, z, e, f = (rnd(rows, 128) for _ in range(5))
    W = rnd(128, 128) / 11
    b = rnd(128)
    s = _act64(z.double(), act).float()
    Wd = W.double()
    y = x.double().mm(Wd if transpose else Wd.t())
    d1, d2 = _derivs64(z.double(), act)
    if act == 0:  # the tanh derivative factors are formed from s as stored
        sd = s.double()
        d1 = 1 - sd * sd
        d2 = -2 * sd * d1

    out0, _ = ops.node_gemm(x, W, transpose=transpose)
    check(out0, y, 1e-6, 'out0', atol_frac=1.0)
    out0, _ = ops.node_gemm(x, W, transpose=transpose, bias=b, residual=r)
    check(out0, y + b.double() + r.double(), 1e-6, 'out0', atol_frac=1.0)
    zz, ss = ops.node_gemm(x, W, transpose=transpose, bias=b, epilogue=ops.NODE_ACT, act=act)
    check(zz, y + b.double(), 1e-6, 'zz', atol_frac=1.0)
    check(ss, _act64(y + b.double(), act), 2e-6, 'ss', atol_frac=1.0)
    _, only = ops.node_gemm(x, W, transpose=transpose, bias=b, epilogue=ops.NODE_ACT, act=act,
                            want_out0=False)
    assert torch.equal(only, ss)
    yy, yd = ops.node_gemm(x, W, transpose=transpose, epilogue=ops.NODE_DACT, act=act, z=z, s=s)
    check(yy, y, 1e-6, 'yy', atol_frac=1.0)
    check(yd, y * d1, 2e-6, 'yd', atol_frac=1.0)
    v, _ = ops.node_gemm(x, W, transpose=transpose, epilogue=ops.NODE_DACT2, act=act, z=z, s=s)
    check(v, y * d1, 2e-6, 'v', atol_frac=1.0)
    v, _ = ops.node_gemm(x, W, transpose=transpose, epilogue=ops.NODE_DACT2, act=act, z=z, s=s,
                         e=e, f=f)
    check(v, y * d1 + e.double() * d2 * f.double(), 2e-6, 'v', atol_frac=1.0)


def test_node_gemm_deterministic_and_checks():
    from mlcg_amd import ops

    x = torch.randn(3000, 128, device="cuda")
    W = torch.randn(128, 128, device="cuda")
    assert torch.equal(ops.node_gemm(x, W)[0], ops.node_gemm(x, W)[0])
    empty = ops.node_gemm(x[:0], W)[0]
    assert empty.shape == (0, 128)
    with pytest.raises(RuntimeError):
        ops.node_gemm(x[:, :64], W[:, :64])
    with pytest.raises(RuntimeError):
        ops.node_gemm(x, W, epilogue=ops.NODE_DACT, act=0)  # z, s missing


@pytest.mark.parametrize("rows", [1, 17, 1000, 17920, 30001])
@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("act", [0, 1])
def test_node_gemm2_matches_two_calls(rows, transpose, act):
    """mlcg_node_gemm2 (two consecutive linears in one kernel) is bitwise the
    pair of mlcg_node_gemm calls it replaces, for every first epilogue, with
    and without the second bias and residual, and checked once against fp64
    torch so that a shared mistake in both paths cannot pass."""
    from mlcg_amd import ops

    print(f"node_gemm2 rows={rows} transpose={transpose} act={act}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows * 4 + 2 * int(transpose) + act + 99)
    rnd = lambda *s: torch.randn(*s, device="cuda", generator=g)  # noqa: E731
    x, r, r2, z, e, f = (rnd(rows, 128) for _ in range(6))
    W, W2 = rnd(128, 128) / 11, rnd(128, 128) / 11
    b, b2 = rnd(128), rnd(128)
    s = _act64(z.double(), act).float()
    kw = dict(transpose=transpose, act=act)

    # ACT then a linear with bias and residual (the interaction block's forward)
    z0, s0 = ops.node_gemm(x, W, bias=b, residual=r, epilogue=ops.NODE_ACT, **kw)
    ref2 = ops.node_gemm(s0, W2, transpose=transpose, bias=b2, residual=r2)[0]
    g0, g1, g2 = ops.node_gemm2(x, W, W2, bias=b, residual=r, epilogue=ops.NODE_ACT,
                                bias2=b2, residual2=r2, **kw)
    assert torch.equal(g0, z0) and torch.equal(g1, s0) and torch.equal(g2, ref2)
    W2d = W2.double()
    y2 = s0.double().mm(W2d if transpose else W2d.t()) + b2.double() + r2.double()
    check(g2, y2, 1e-6, 'g2', atol_frac=1.0)
    g0, g1, g2 = ops.node_gemm2(x, W, W2, bias=b, epilogue=ops.NODE_ACT, want_out0=False, **kw)
    z0, s0 = ops.node_gemm(x, W, bias=b, epilogue=ops.NODE_ACT, **kw)
    assert g0 is None and torch.equal(g1, s0)
    assert torch.equal(g2, ops.node_gemm(s0, W2, transpose=transpose)[0])

    # DACT then a linear (reverse and tangent sweeps), with and without residual
    y0, v0 = ops.node_gemm(x, W, epilogue=ops.NODE_DACT, z=z, s=s, **kw)
    for res2 in (None, r2):
        g0, g1, g2 = ops.node_gemm2(x, W, W2, epilogue=ops.NODE_DACT, z=z, s=s, residual2=res2,
                                    **kw)
        assert torch.equal(g0, y0) and torch.equal(g1, v0)
        assert torch.equal(g2, ops.node_gemm(v0, W2, transpose=transpose, residual=res2)[0])

    # DACT2 (with and without the e, f term) then a linear (double backward)
    for ef in ((None, None), (e, f)):
        v0, _ = ops.node_gemm(x, W, epilogue=ops.NODE_DACT2, z=z, s=s, e=ef[0], f=ef[1], **kw)
        g0, g1, g2 = ops.node_gemm2(x, W, W2, epilogue=ops.NODE_DACT2, z=z, s=s, e=ef[0],
                                    f=ef[1], **kw)
        assert g1 is None and torch.equal(g0, v0)
        assert torch.equal(g2, ops.node_gemm(v0, W2, transpose=transpose)[0])


@pytest.mark.parametrize("rows", [1, 17, 1000, 17920])
@pytest.mark.parametrize("transpose", [False, True])
def test_node_weight_images_bit_identical(rows, transpose):
    """Products that read pre-split weight images (mlcg_node_weight_images)
    equal those that split the weights in the kernel, bit for bit, for every
    epilogue of node_gemm and node_gemm2; an image of the other orientation
    gives a different product, so the orientation is part of the image; a
    malformed image raises."""
    from mlcg_amd import ops

    print(f"weight images rows={rows} transpose={transpose}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows * 2 + int(transpose) + 7)
    rnd = lambda *s: torch.randn(*s, device="cuda", generator=g)  # noqa: E731
    x, r, z, e, f = (rnd(rows, 128) for _ in range(5))
    s = torch.tanh(z)
    W, W2 = rnd(128, 128) / 11, rnd(128, 128) * 3
    b = rnd(128)
    imgs = ops.node_weight_images([W, W2, W], [transpose, transpose, not transpose])
    assert imgs.shape == (3, ops.NODE_W_IMAGE_HALFS) and imgs.dtype == torch.float16
    wi, w2i, other = imgs[0], imgs[1], imgs[2]
    kw = dict(transpose=transpose, act=0)
    for ep, extra in ((ops.NODE_PLAIN, dict(bias=b, residual=r)),
                      (ops.NODE_ACT, dict(bias=b)),
                      (ops.NODE_DACT, dict(z=z, s=s)),
                      (ops.NODE_DACT2, dict(z=z, s=s, e=e, f=f))):
        ref = ops.node_gemm(x, W, epilogue=ep, **kw, **extra)
        got = ops.node_gemm(x, W, epilogue=ep, w_image=wi, **kw, **extra)
        for a_, c_ in zip(ref, got):
            assert (a_ is None and c_ is None) or torch.equal(a_, c_), ep
        if ep != ops.NODE_PLAIN:
            ref2 = ops.node_gemm2(x, W, W2, epilogue=ep, residual2=r, **kw, **extra)
            for images in ((wi, None), (None, w2i), (wi, w2i)):
                got2 = ops.node_gemm2(x, W, W2, epilogue=ep, residual2=r, w_image=images[0],
                                      w2_image=images[1], **kw, **extra)
                for a_, c_ in zip(ref2, got2):
                    assert (a_ is None and c_ is None) or torch.equal(a_, c_), (ep, images)
    if rows >= 17:
        wrong = ops.node_gemm(x, W, transpose=transpose, w_image=other)[0]
        assert not torch.equal(wrong, ops.node_gemm(x, W, transpose=transpose)[0])
    with pytest.raises(RuntimeError, match="image"):
        ops.node_gemm(x, W, w_image=wi[:100])
    with pytest.raises(RuntimeError, match="image"):
        ops.node_gemm(x, W, w_image=wi.float())


def test_node_gemm2_checks():
    from mlcg_amd import ops

    x = torch.randn(100, 128, device="cuda")
    W = torch.randn(128, 128, device="cuda")
    out = ops.node_gemm2(x[:0], W, W, epilogue=ops.NODE_ACT)
    assert out[2].shape == (0, 128)
    with pytest.raises(RuntimeError):
        ops.node_gemm2(x, W, W, epilogue=ops.NODE_PLAIN)
    with pytest.raises(RuntimeError):
        ops.node_gemm2(x, W, W[:, :64], epilogue=ops.NODE_ACT)
    with pytest.raises(RuntimeError):
        ops.node_gemm2(x, W, W, epilogue=ops.NODE_DACT, act=0)  # z, s missing


@pytest.mark.gpu
@pytest.mark.parametrize("rows,num_types", [(0, 5), (1, 1), (17920, 35), (17920, 100),
                                            (5000, 128), (300, 7), (24576, 3), (24577, 3),
                                            (50000, 1), (200000, 3), (128000, 20)])
def test_type_sum_matches_index_add(rows, num_types):
    """The embedding-table gradient against fp64 index_add, identical on
    repeated calls (fixed summation order)."""
    from mlcg_amd import ops

    print(f"type_sum rows={rows} num_types={num_types}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows + num_types)
    x = torch.randn(rows, 128, device="cuda", generator=g)
    types = torch.randint(0, num_types, (rows,), device="cuda", generator=g)
    out, bad = ops.type_sum(x, types, num_types)
    ref = torch.zeros(num_types, 128, dtype=torch.float64).index_add_(
        0, types.cpu(), x.double().cpu())
    assert int(bad.item()) == 0
    if rows == 0:
        assert torch.equal(out.cpu(), torch.zeros(num_types, 128))
    else:
        check(out, ref, 1e-6, 'out', atol_frac=1.0)
    assert torch.equal(ops.type_sum(x, types, num_types)[0], out)


@pytest.mark.gpu
def test_type_sum_sorted_and_skewed_types():
    """Row lists that cross the 24,576-row chunks unevenly: all rows of one
    type in a block at the end, and types sorted ascending (frames of a
    batch), against fp64 index_add."""
    from mlcg_amd import ops

    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(40000, 128, device="cuda", generator=g)
    types = torch.zeros(40000, dtype=torch.int64, device="cuda")
    types[-20000:] = 2
    for tt in (types, torch.sort(torch.randint(0, 50, (40000,), device="cuda",
                                               generator=g))[0]):
        out, bad = ops.type_sum(x, tt, 50)
        ref = torch.zeros(50, 128, dtype=torch.float64).index_add_(0, tt.cpu(), x.double().cpu())
        assert int(bad.item()) == 0
        check(out, ref, 1e-6, 'out', atol_frac=1.0)


@pytest.mark.gpu
def test_type_sum_flags_out_of_table_types():
    from mlcg_amd import ops

    x = torch.ones(10, 128, device="cuda")
    types = torch.tensor([0, 1, 2, 3, 9, 1, 1, 0, 2, 3], device="cuda")
    ops.numerics_flags(clear=True)
    out, bad = ops.type_sum(x, types, 4)
    assert int(bad.item()) == 1
    assert out[:, 0].tolist() == [2.0, 3.0, 2.0, 2.0]  # the type-9 row is skipped
    ops.check_numerics()  # reported in bad, not in the flags
    out2, none = ops.type_sum(x, types, 4, want_bad=False)
    assert none is None and torch.equal(out2, out)
    with pytest.raises(RuntimeError, match="embedding table"):
        ops.check_numerics()
    assert ops.type_sum(x, types.clamp(max=3), 4, want_bad=False)[1] is None
    ops.check_numerics()
    with pytest.raises(RuntimeError):
        ops.type_sum(x, types, 129)


def test_copy_batch():
    """One launch copies up to eight tensors (sizes not a multiple of 16
    bytes included); more pairs take one launch per eight; mismatched pairs
    raise before anything is launched."""
    from mlcg_amd import ops

    g = torch.Generator(device="cuda").manual_seed(8)
    srcs = [torch.randn(17920, 3, device="cuda", generator=g),
            torch.randint(0, 9, (17920,), device="cuda", generator=g),
            torch.randint(0, 9, (3,), device="cuda", generator=g),
            torch.randn(5, device="cuda", generator=g),
            torch.empty(0, device="cuda"),
            torch.randint(0, 2 ** 30, (7, 5), dtype=torch.int32, device="cuda", generator=g),
            torch.randn(1000, 128, device="cuda", generator=g).half(),
            torch.randn(1, device="cuda", generator=g).double(),
            torch.randn(33, 3, device="cuda", generator=g),
            torch.randn(2, device="cuda", generator=g)]
    for n in (1, 8, 10):
        dsts = [torch.full_like(t, 7) for t in srcs[:n]]
        ops.copy_batch(dsts, srcs[:n])
        for d, t in zip(dsts, srcs[:n]):
            assert torch.equal(d, t)
    with pytest.raises(RuntimeError, match="copy_batch"):
        ops.copy_batch([torch.empty(4, device="cuda")], [torch.empty(5, device="cuda")])
    with pytest.raises(RuntimeError, match="copy_batch"):
        ops.copy_batch([torch.empty(8, device="cuda")[1:5]], [torch.empty(4, device="cuda")])


@pytest.mark.parametrize("rows", [1, 33, 17920, 128000])
def test_embedding_gather(rows):
    """The embedding lookup equals torch's index_select bit for bit; a type
    outside the table gives a zero row and raises through check_numerics."""
    from mlcg_amd import ops

    print(f"embedding_gather rows={rows}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows)
    table = torch.randn(100, 128, device="cuda", generator=g)
    types = torch.randint(0, 100, (rows,), device="cuda", generator=g)
    ops.numerics_flags(clear=True)
    assert torch.equal(ops.embedding_gather(table, types), table.index_select(0, types))
    ops.check_numerics()
    bad = types.clone()
    bad[rows // 2] = 100
    out = ops.embedding_gather(table, bad)
    assert float(out[rows // 2].abs().max()) == 0.0
    keep = torch.arange(rows, device="cuda") != rows // 2
    assert torch.equal(out[keep], table.index_select(0, types)[keep])
    with pytest.raises(RuntimeError, match="embedding table"):
        ops.check_numerics()
