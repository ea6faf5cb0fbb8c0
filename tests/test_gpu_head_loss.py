"""ane_head_loss: the classifier-head cross-entropy on caller-owned device
buffers (torch tensors serve as plain device memory here), against a
float64 log-sum-exp / cross-entropy of the same fp16 operands, with the
reference's rules: targets >= vocab excluded, p clamped at 1e-10
(ane/stories/cpu.go:212-292), optional 15*tanh softcap."""
import ctypes as C

import numpy as np
import pytest

from ane import _lib

pytestmark = pytest.mark.gpu


def _ptr(t):
    return C.c_void_p(t.data_ptr())


def reference(xn, embed, tg, seq, softcap):
    lg = embed.astype(np.float64) @ xn.astype(np.float64).T           # [V, T]
    if softcap:
        lg = 15.0 * np.tanh(lg / 15.0)
    m = lg.max(0)
    lse = m + np.log(np.exp(lg - m).sum(0))
    V, T = lg.shape
    ok = tg < V
    tok = np.zeros(T)
    idx = np.nonzero(ok)[0]
    tok[idx] = np.minimum(lse[idx] - lg[tg[idx].astype(np.int64), idx], -np.log(1e-10))
    per = []
    for b in range(T // seq):
        s = slice(b * seq, (b + 1) * seq)
        n = ok[s].sum()
        per.append(tok[s][ok[s]].sum() / n if n else 0.0)
    return np.array(per), lse


def run(lib, torch, xn, embed, tg, seq, softcap, with_lse=True):
    dev = torch.device("cuda")
    x_d = torch.from_numpy(xn.view(np.int16).copy()).to(dev)
    e_d = torch.from_numpy(embed.view(np.int16).copy()).to(dev)
    t_d = torch.from_numpy(tg.view(np.int16).copy()).to(dev)
    T, D = xn.shape
    V = embed.shape[0]
    loss = torch.full((T // seq,), float("nan"), dtype=torch.float32, device=dev)
    lse = torch.full((T,), float("nan"), dtype=torch.float32, device=dev) if with_lse else None
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.ane_head_loss(_ptr(x_d), _ptr(e_d), _ptr(t_d), T, D, V, seq, softcap, _ptr(loss),
                           _ptr(lse) if lse is not None else None, stream)
    assert rc == 0, lib.ane_op_last_error()
    torch.cuda.synchronize()
    return loss.cpu().numpy(), (lse.cpu().numpy() if lse is not None else None)


# tiles: 128x64 at 192 and 512 tokens, the 8-wave 256x256 from 1024 tokens
@pytest.mark.parametrize("T,seq,softcap", [(512, 256, 0), (512, 128, 1), (1024, 256, 0), (192, 64, 1)])
def test_head_loss_matches_f64(T, seq, softcap):
    torch = pytest.importorskip("torch")
    lib = _lib.load()
    V, D = 32000, 768
    r = np.random.default_rng(T + seq + softcap)
    xn = r.standard_normal((T, D)).astype(np.float16)
    embed = (r.standard_normal((V, D)) * (0.3 if softcap else 0.05)).astype(np.float16)
    tg = r.integers(0, V, T).astype(np.uint16)
    tg[5] = V                  # excluded
    if T // seq > 2:
        tg[seq:2 * seq] = 65535    # a sequence with no valid target: loss 0
    per, lse = run(lib, torch, xn, embed, tg, seq, softcap)
    ref_per, ref_lse = reference(xn, embed, tg, seq, softcap)
    np.testing.assert_allclose(lse, ref_lse, rtol=0, atol=2e-4)
    np.testing.assert_allclose(per, ref_per, rtol=0, atol=1e-4)
    per2, _ = run(lib, torch, xn, embed, tg, seq, softcap, with_lse=False)
    np.testing.assert_array_equal(per2, per)


def test_head_loss_errors():
    torch = pytest.importorskip("torch")
    lib = _lib.load()
    buf = torch.zeros(64, dtype=torch.float32, device="cuda")
    p = _ptr(buf)
    assert lib.ane_head_loss(p, p, p, 100, 64, 64, 100, 0, p, None, None) == _lib.ANE_ERR_ARG
    assert b"ntok=100" in lib.ane_op_last_error()
    assert lib.ane_head_loss(None, p, p, 64, 64, 64, 64, 0, p, None, None) == _lib.ANE_ERR_ARG
