"""Shared builders for the tests (model from a reference-layout state_dict,
synthetic batches on a device, error metrics)."""

import torch

from oracle import schnet_ref as R


def make_cfg(num_blocks=3, num_rbf=50, rc=20.0, act="tanh", rbf_cut="cosine",
             conv_cut="cosine", conv_lo=0.0, basis="gaussian", aggr="add"):
    return R.SchNetConfig(num_rbf=num_rbf, rbf_lo=0.0, rbf_hi=rc, rbf_cut=rbf_cut,
                          conv_cut=conv_cut, conv_lo=conv_lo, conv_hi=rc, act=act,
                          num_blocks=num_blocks, basis=basis, aggr=aggr)


def make_model(cfg, sd, out_widths=(64,), device="cuda", trainable_basis=False):
    from mlcg_amd import nn

    act = torch.nn.Tanh() if cfg.act == "tanh" else nn.ShiftedSoftplus()
    rbf_cut = (nn.CosineCutoff(0.0, cfg.rbf_hi) if cfg.rbf_cut == "cosine"
               else nn.IdentityCutoff(0.0, cfg.rbf_hi))
    conv_cut = (nn.CosineCutoff(cfg.conv_lo, cfg.conv_hi) if cfg.conv_cut == "cosine"
                else nn.IdentityCutoff(cfg.conv_lo, cfg.conv_hi))
    if cfg.basis == "gaussian":
        rbf = nn.GaussianBasis(rbf_cut, num_rbf=cfg.num_rbf, trainable=trainable_basis)
    else:
        rbf = nn.ExpNormalBasis(rbf_cut, num_rbf=cfg.num_rbf, trainable=trainable_basis)
    m = nn.StandardSchNet(rbf, conv_cut, list(out_widths), hidden_channels=128,
                          embedding_size=sd["embedding_layer.weight"].shape[0],
                          num_filters=128, num_interactions=cfg.num_blocks, activation=act,
                          aggr=getattr(cfg, "aggr", "add"))
    m.load_state_dict(sd)
    return m.to(device)


def rel_err(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def max_abs(a, b):
    return float((a.double().cpu() - b.double().cpu()).abs().max())


def close_report(got, ref, rtol, atol):
    """Element-wise check |got - ref| <= atol + rtol * |ref| (torch.allclose's
    rule) in fp64.  Returns (n_fail, n, worst ratio |d| / (atol + rtol |ref|),
    a description of the worst element)."""
    a = got.detach().double().cpu().reshape(-1)
    r = ref.detach().double().cpu().reshape(-1)
    if a.numel() == 0:
        return 0, 0, 0.0, "empty"
    d = (a - r).abs()
    lim = atol + rtol * r.abs()
    ratio = torch.where(lim > 0, d / lim.clamp_min(1e-300),
                        torch.where(d > 0, torch.full_like(d, float("inf")), torch.zeros_like(d)))
    ratio = torch.where(torch.isfinite(a), ratio, torch.full_like(d, float("inf")))
    k = int(torch.argmax(ratio))
    n_fail = int((ratio > 1.0).sum())
    desc = (f"worst at flat index {k}: got {float(a[k]):.9e} ref {float(r[k]):.9e} "
            f"|d| {float(d[k]):.3e} ratio {float(ratio[k]):.3f}; max|d| {float(d.max()):.3e}, "
            f"max|ref| {float(r.abs().max()):.3e}")
    return n_fail, a.numel(), float(ratio[k]), desc


def assert_close(got, ref, rtol, atol, name=""):
    """Element-wise parity assertion: every element within atol + rtol |ref|.
    Prints the worst element (so a passing run still shows the margin)."""
    assert tuple(got.shape) == tuple(ref.shape), (name, tuple(got.shape), tuple(ref.shape))
    n_fail, n, worst, desc = close_report(got, ref, rtol, atol)
    print(f"{name}: rtol {rtol:g} atol {atol:.3g}: {n_fail}/{n} outside; {desc}")
    assert n_fail == 0, f"{name}: {n_fail}/{n} elements outside rtol {rtol:g} atol {atol:.3g}; {desc}"
    return worst


def scaled_atol(ref, scale):
    """An absolute tolerance of `scale` times the largest |ref| element."""
    return scale * float(ref.detach().double().abs().max()) if ref.numel() else 0.0


def check(got, ref, rtol, name="", atol_frac=0.1):
    """assert_close with the absolute term atol_frac * rtol times the largest
    |ref| element: every element within rtol of itself, or within
    atol_frac * rtol of the tensor's scale (elements near zero are sums of
    cancelling terms, whose fp32 rounding error scales with the terms, not with
    the sum).  atol_frac = 0.1 for model outputs (energies, forces, parameter
    gradients); 1.0 -- every element within rtol of the tensor's largest, a
    max-norm relative bound -- where a test says why."""
    return assert_close(got, ref, rtol, scaled_atol(ref, atol_frac * rtol), name)


def check_calibrated(got, ref, ref32, rtol, name="", atol_frac=0.1):
    """check() with the bound widened, where needed, to twice the error of the
    reference's own fp32 arithmetic on the same inputs (`ref32`: the oracle
    evaluated in fp32, op for op as the reference): every element within
    max(1, 2 r32) x (atol + rtol |ref|), r32 being the fp32 oracle's worst
    ratio.  On small, cancellation-heavy test models the fp32 reference itself
    misses the north_star bar by a little; the kernels must then be no worse
    than twice the reference."""
    atol = scaled_atol(ref, atol_frac * rtol)
    r32 = close_report(ref32, ref, rtol, atol)[2]
    scale = max(1.0, 2.0 * r32)
    print(f"{name}: reference fp32 arithmetic ratio {r32:.3f} -> bound x{scale:.3f}")
    return assert_close(got, ref, rtol * scale, atol * scale, name)
