"""Independent float64 PyTorch model used to pin the C oracle on small shapes.

Written token-major with torch primitives (scaled_dot_product_attention,
cross_entropy, autograd) so that it shares no code with oracle/refcpu.c.
Gradients come from autograd.  The reference's compat-mode backward
quirks are expressed as straight-through substitutions whose VALUE is the
forward of the reference and whose GRADIENT is what the reference's
backward computes:

* attention backward recomputes probabilities with scale 1.0
  (ane/train_full.go:268-269): out = A_1 + (A_{1/8} - A_1).detach()
* no RoPE backward (ane/train_full.go:646-665): q_rot = q + (rope(q) - q).detach()
* QK-norm backward scales the projection term by 1.2^2 (ane/common.go:247):
  y = s*q*r.detach() + s^2*(q.detach()*r - q.detach()*r.detach())
* the x0 gradient is added before smear backward (ane/train_full.go:790-798):
  x0_used = x_smeared + (x0 - x_smeared).detach()
"""
import math

import numpy as np
import torch
import torch.nn.functional as F

EPS = 1e-5


def rms(x):
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + EPS)


def rope(x, heads, theta):
    # x [S, D]; interleaved pairs (2i, 2i+1) within each head
    S, D = x.shape
    hd = D // heads
    pos = torch.arange(S, dtype=torch.float64)[:, None]
    i = torch.arange(hd // 2, dtype=torch.float64)[None, :]
    ang = pos / (theta ** (2 * i / hd))
    c, s = torch.cos(ang), torch.sin(ang)
    xr = x.view(S, heads, hd // 2, 2)
    e, o = xr[..., 0], xr[..., 1]
    c = c[:, None, :]
    s = s[:, None, :]
    return torch.stack([e * c - o * s, o * c + e * s], -1).reshape(S, D)


def qknorm(x, heads, compat):
    S, D = x.shape
    hd = D // heads
    xh = x.view(S, heads, hd)
    r = torch.rsqrt((xh * xh).mean(-1, keepdim=True) + EPS)
    s = 1.2
    if not compat:
        return (s * xh * r).reshape(S, D)
    y = s * xh * r.detach() + s * s * (xh.detach() * r - xh.detach() * r.detach())
    return y.reshape(S, D)


def attention(q, k, v, heads, scale):
    S, D = q.shape
    hd = D // heads
    qh = q.view(S, heads, hd).transpose(0, 1)
    kh = k.view(S, heads, hd).transpose(0, 1)
    vh = v.view(S, heads, hd).transpose(0, 1)
    o = F.scaled_dot_product_attention(qh, kh, vh, is_causal=True, scale=scale)
    return o.transpose(0, 1).reshape(S, D)


def model_loss(cfg, P, tokens, targets, grad_mode="true"):
    """P: dict name -> float64 tensor (requires_grad as wanted).
    tokens/targets: int64 [B, S].  Returns (mean loss, logits [B,S,V])."""
    nano = cfg.arch == "nanochat"
    compat = nano and grad_mode == "compat"
    L, NH, D = cfg.layers, cfg.heads, cfg.dim
    hd = D // NH
    losses, all_logits = [], []
    for b in range(tokens.shape[0]):
        tok = tokens[b]
        x = P["embed"][tok]
        if nano:
            x = rms(x)
            x0 = x
            g = torch.sigmoid(x @ P["smear_gate"].T)
            shifted = torch.cat([torch.zeros_like(x[:1]), x[:-1]], 0)
            x = x + P["smear_lambda"][0] * g * shifted
            x0u = x + (x0 - x).detach() if compat else x0
        xmid = None
        for l in range(L):
            pre = f"layers.{l}."
            xn = rms(x) * P[pre + "g_att"] if not nano else rms(x)
            q = xn @ P[pre + "wq"].T
            k = xn @ P[pre + "wk"].T
            v = xn @ P[pre + "wv"].T
            qr, kr = rope(q, NH, cfg.rope_theta), rope(k, NH, cfg.rope_theta)
            if compat:
                qr = q + (qr - q).detach()
                kr = k + (kr - k).detach()
            if nano:
                qr, kr = qknorm(qr, NH, compat), qknorm(kr, NH, compat)
            if (pre + "ve_embed") in P:
                gate = torch.sigmoid(x[:, :12] @ P[pre + "ve_gate"].view(NH, 12).T)  # [S, NH]
                ve = P[pre + "ve_embed"][tok]
                v = v + (3.0 * gate[:, :, None] * ve.view(-1, NH, hd)).reshape(-1, D)
            if compat:
                a1 = attention(qr, kr, v, NH, 1.0)
                a8 = attention(qr, kr, v, NH, 1.0 / math.sqrt(hd))
                att = a1 + (a8 - a1).detach()
            else:
                att = attention(qr, kr, v, NH, 1.0 / math.sqrt(hd))
            if nano:
                rl, xl = P["resid_lambdas"][l], P["x0_lambdas"][l]
                x2 = rl * x + att @ P[pre + "wo"].T + xl * x0u
                xn2 = rms(x2)
                h = torch.relu(xn2 @ P[pre + "w1"].T) ** 2
                x = rl * x2 + h @ P[pre + "w2"].T + xl * x0u
            else:
                x2 = x + att @ P[pre + "wo"].T
                xn2 = rms(x2) * P[pre + "g_ffn"]
                h = F.silu(xn2 @ P[pre + "w1"].T) * (xn2 @ P[pre + "w3"].T)
                x = x2 + h @ P[pre + "w2"].T
            if nano and l == L // 2 - 1:
                xmid = x
        if nano:
            x = x - P["backout_lambda"][0] * xmid
            xn = rms(x)
        else:
            xn = rms(x) * P["g_final"]
        logits = xn @ P["embed"].T
        if nano:
            logits = 15.0 * torch.tanh(logits / 15.0)
        valid = targets[b] < cfg.vocab
        loss = F.cross_entropy(logits[valid], targets[b][valid])
        losses.append(loss)
        all_logits.append(logits)
    return torch.stack(losses).mean(), torch.stack(all_logits)


def params_to_torch(cfg, flat, requires_grad=True):
    import ane
    out = {}
    for name, arr in ane.views(cfg, flat).items():
        t = torch.tensor(np.array(arr, dtype=np.float64))
        t.requires_grad_(requires_grad)
        out[name] = t
    return out


def grads_flat(cfg, P):
    import ane
    g = np.zeros(ane.param_count(cfg), np.float64)
    for name, off, shape in ane.param_layout(cfg):
        t = P[name]
        if t.grad is not None:
            g[off:off + t.numel()] = t.grad.detach().numpy().reshape(-1)
    return g


def gqa_logits(cfg, P, tokens):
    """Full causal forward of the Llama2-style model with grouped-query
    attention (key/value head h // (heads // kv_heads) serves query head h),
    float64.  tokens: int64 [B, S]; returns logits [B, S, V]."""
    NH, NKV, D = cfg.heads, cfg.kv_heads, cfg.dim
    hd = D // NH
    out = []
    for b in range(tokens.shape[0]):
        tok = tokens[b]
        S = tok.shape[0]
        x = P["embed"][tok]
        for l in range(cfg.layers):
            pre = f"layers.{l}."
            xn = rms(x) * P[pre + "g_att"]
            q = rope(xn @ P[pre + "wq"].T, NH, cfg.rope_theta)
            k = rope(xn @ P[pre + "wk"].T, NKV, cfg.rope_theta)
            v = xn @ P[pre + "wv"].T
            rep = NH // NKV
            kf = k.view(S, NKV, hd).repeat_interleave(rep, dim=1).reshape(S, D)
            vf = v.view(S, NKV, hd).repeat_interleave(rep, dim=1).reshape(S, D)
            att = attention(q, kf, vf, NH, 1.0 / math.sqrt(hd))
            x = x + att @ P[pre + "wo"].T
            xn2 = rms(x) * P[pre + "g_ffn"]
            x = x + (F.silu(xn2 @ P[pre + "w1"].T) * (xn2 @ P[pre + "w3"].T)) @ P[pre + "w2"].T
        out.append((rms(x) * P["g_final"]) @ P["embed"].T)
    return torch.stack(out)
