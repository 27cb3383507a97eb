"""Shared builders for the tests (model from a reference-layout state_dict,
synthetic batches on a device, error metrics)."""

import torch

from oracle import schnet_ref as R


def make_cfg(num_blocks=3, num_rbf=50, rc=20.0, act="tanh", rbf_cut="cosine",
             conv_cut="cosine", conv_lo=0.0, basis="gaussian"):
    return R.SchNetConfig(num_rbf=num_rbf, rbf_lo=0.0, rbf_hi=rc, rbf_cut=rbf_cut,
                          conv_cut=conv_cut, conv_lo=conv_lo, conv_hi=rc, act=act,
                          num_blocks=num_blocks, basis=basis)


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
                          num_filters=128, num_interactions=cfg.num_blocks, activation=act)
    m.load_state_dict(sd)
    return m.to(device)


def rel_err(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def max_abs(a, b):
    return float((a.double().cpu() - b.double().cpu()).abs().max())
