"""Writes tests/golden/*.npz: float64 torch-CPU references for the oracle.

The networks, losses and optimiser step are written here with torch library
routines (F.layer_norm, matmul, log_softmax, autograd, clip_grad_norm_,
torch.optim.Adam), independently of the oracle's hand-written loops and
gradients, on small random inputs. Run from the repo root:

    python tests/golden/make_golden.py
"""
import math
import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
LOG_SQRT_2PI = 0.5 * math.log(2.0 * math.pi)


def pad128(x):
    return (x + 127) // 128 * 128


def layout(O, A, E, H, L, continuous):
    """Canonical flat layout: vector parameters first, then matrices, each padded to 128."""
    off, o = {}, 0
    off["in_w"], o = o, o + pad128(O * E)
    off["in_b"], o = o, o + pad128(E)
    for l in range(L + 1):
        off[f"g{l}"], o = o, o + pad128(E)
        off[f"b{l}"], o = o, o + pad128(E)
    if continuous:
        off["log_std"], o = o, o + pad128(A)
    for l in range(L):
        off[f"up{l}"], o = o, o + pad128(E * H)
        off[f"down{l}"], o = o, o + pad128(H * E)
    off["head"], o = o, o + pad128(E * (A + 1))
    return off, o


def shapes(O, A, E, H, L, continuous):
    s = {"in_w": (O, E), "in_b": (E,), "head": (E, A + 1)}
    for l in range(L + 1):
        s[f"g{l}"] = (E,)
        s[f"b{l}"] = (E,)
    for l in range(L):
        s[f"up{l}"] = (E, H)
        s[f"down{l}"] = (H, E)
    if continuous:
        s["log_std"] = (A,)
    return s


def random_params(rs, O, A, E, H, L, continuous):
    off, count = layout(O, A, E, H, L, continuous)
    flat = np.zeros(count, np.float32)
    for k, shp in shapes(O, A, E, H, L, continuous).items():
        n = int(np.prod(shp))
        if k.startswith("g"):
            v = 1.0 + 0.1 * rs.standard_normal(n)
        elif k.startswith("b") or k == "in_b":
            v = 0.1 * rs.standard_normal(n)
        elif k == "log_std":
            v = 0.3 * rs.standard_normal(n)
        else:
            v = rs.standard_normal(n) / math.sqrt(shp[0])
        flat[off[k]:off[k] + n] = v.astype(np.float32)
    return flat


def torch_params(flat, O, A, E, H, L, continuous):
    off, _ = layout(O, A, E, H, L, continuous)
    t = {}
    for k, shp in shapes(O, A, E, H, L, continuous).items():
        n = int(np.prod(shp))
        t[k] = torch.tensor(flat[off[k]:off[k] + n].astype(np.float64).reshape(shp), requires_grad=True)
    return t


def forward(t, obs, E, L):
    h = obs @ t["in_w"] + t["in_b"]
    for l in range(L):
        x = F.layer_norm(h, (E,), t[f"g{l}"], t[f"b{l}"], eps=1e-5)
        h = h + torch.relu(x @ t[f"up{l}"]) @ t[f"down{l}"]
    x = F.layer_norm(h, (E,), t[f"g{L}"], t[f"b{L}"], eps=1e-5)
    return x @ t["head"]


def ppo_loss(head, A, continuous, t, actions, adv, ret, old_logp, clip, vc, ec):
    an = (adv - adv.mean()) / (torch.sqrt(((adv - adv.mean()) ** 2).mean()) + 1e-8)
    value = head[:, A]
    if continuous:
        mu = head[:, :A]
        ls = t["log_std"]
        d = (actions - mu) * torch.exp(-ls)
        logp = (-0.5 * d * d - ls - LOG_SQRT_2PI).sum(-1)
        entropy = (ls + LOG_SQRT_2PI + 0.5).sum().expand(head.shape[0])
    else:
        lp_all = torch.log_softmax(head[:, :A], dim=-1)
        entropy = -(torch.exp(lp_all) * lp_all).sum(-1)
        logp = lp_all.gather(1, actions.view(-1, 1)).squeeze(1)
    ratio = torch.exp(logp - old_logp)
    s1 = ratio * an
    s2 = torch.clamp(ratio, 1 - clip, 1 + clip) * an
    pol = -torch.where(s1 <= s2, s1, s2)
    vloss = 0.5 * vc * (value - ret) ** 2
    loss = (pol + vloss - ec * entropy).mean()
    stats = [pol.mean(), vloss.mean(), entropy.mean(), (old_logp - logp).mean(),
             ((ratio - 1).abs() > clip).double().mean()]
    return loss, logp, stats


def make_case(name, seed, O, A, E, H, L, B, continuous, steps=3):
    rs = np.random.default_rng(seed)
    flat = random_params(rs, O, A, E, H, L, continuous)
    obs = (rs.standard_normal((B, O)) * 1.5).astype(np.float32)
    adv = rs.standard_normal(B).astype(np.float32) * 2 + 0.5
    ret = rs.standard_normal(B).astype(np.float32)
    clip, vc, ec, mgn, lr = 0.2, 0.5, 0.01, 0.5, 3e-4
    t = torch_params(flat, O, A, E, H, L, continuous)
    with torch.no_grad():
        head0 = forward(t, torch.tensor(obs, dtype=torch.float64), E, L)
    if continuous:
        actions = (head0[:, :A].numpy() + rs.standard_normal((B, A))).astype(np.float32)
        act_t = torch.tensor(actions, dtype=torch.float64)
    else:
        actions = rs.integers(0, A, B).astype(np.int32)
        act_t = torch.tensor(actions, dtype=torch.int64)
    # old log-probs near the current ones, so some ratios leave the clip band
    with torch.no_grad():
        _, lp0, _ = ppo_loss(head0, A, continuous, t, act_t, torch.tensor(adv, dtype=torch.float64),
                             torch.tensor(ret, dtype=torch.float64), torch.zeros(B, dtype=torch.float64), clip, vc,
                             ec)
    old_logp = (lp0.numpy() + 0.3 * rs.standard_normal(B)).astype(np.float32)

    obs_t = torch.tensor(obs, dtype=torch.float64)
    adv_t, ret_t, old_t = (torch.tensor(x, dtype=torch.float64) for x in (adv, ret, old_logp))
    params = list(t.values())
    opt = torch.optim.Adam(params, lr=lr, betas=(0.9, 0.999), eps=1e-8)
    off, count = layout(O, A, E, H, L, continuous)
    out = {"dims": np.array([O, A, E, H, L, int(continuous), B], np.int64),
           "hp": np.array([clip, vc, ec, mgn, 0.99, 0.95, lr], np.float64),
           "params0": flat, "obs": obs, "actions": actions, "adv": adv, "ret": ret, "old_logp": old_logp,
           "head0": head0.numpy().astype(np.float32)}
    for s in range(steps):
        opt.zero_grad()
        head = forward(t, obs_t, E, L)
        loss, _, st = ppo_loss(head, A, continuous, t, act_t, adv_t, ret_t, old_t, clip, vc, ec)
        loss.backward()
        g = np.zeros(count, np.float64)
        for k, v in t.items():
            n = v.numel()
            g[off[k]:off[k] + n] = v.grad.numpy().ravel()
        norm = float(torch.nn.utils.clip_grad_norm_(params, mgn))
        opt.step()
        p = np.zeros(count, np.float64)
        for k, v in t.items():
            n = v.numel()
            p[off[k]:off[k] + n] = v.detach().numpy().ravel()
        out[f"grad{s}"] = g.astype(np.float32)
        out[f"params{s + 1}"] = p.astype(np.float32)
        out[f"stats{s}"] = np.array([x.item() for x in st] + [norm], np.float64)
        out[f"head{s}"] = head.detach().numpy().astype(np.float32)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)
    print(name, count, "params")


if __name__ == "__main__":
    torch.manual_seed(0)
    make_case("ppo_categorical", 1, O=4, A=3, E=32, H=64, L=2, B=64, continuous=False)
    make_case("ppo_gaussian", 2, O=5, A=2, E=32, H=32, L=1, B=48, continuous=True)
    make_case("ppo_voxel_shape", 3, O=30, A=6, E=32, H=64, L=2, B=64, continuous=False, steps=1)
