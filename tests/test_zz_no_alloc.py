"""ane_head_loss_noalloc, the allocation-free form of ane_head_loss (its
scratch is a fixed per-GPU array), against ane_head_loss through the C-ABI:
two calls in a row, the second smaller, each equal to the allocating
entry's result; free device memory does not change across the calls; sizes
past the array are refused with a clear error."""
import ctypes as C

import numpy as np
import pytest

from ane import _lib

pytestmark = pytest.mark.gpu


def _ptr(t):
    return C.c_void_p(t.data_ptr())


def _case(torch, T, seq, softcap, seed):
    V, D = 32000, 768
    r = np.random.default_rng(seed)
    dev = torch.device("cuda")
    xn = torch.from_numpy(r.standard_normal((T, D)).astype(np.float16).view(np.int16)).to(dev)
    embed = torch.from_numpy((r.standard_normal((V, D)) * 0.05).astype(np.float16).view(np.int16)).to(dev)
    tg = r.integers(0, V, T).astype(np.uint16)
    tg[3] = 65535
    return xn, embed, torch.from_numpy(tg.view(np.int16)).to(dev), T, D, V, seq, softcap


def _outputs(torch, case):
    T, seq = case[3], case[6]
    return (torch.full((T // seq,), float("nan"), dtype=torch.float32, device="cuda"),
            torch.full((T,), float("nan"), dtype=torch.float32, device="cuda"))


def _run(lib, torch, fn, case, outs, with_lse=True):
    xn, embed, tg, T, D, V, seq, softcap = case
    loss, lse = outs
    loss.fill_(float("nan"))
    lse.fill_(float("nan"))
    if not with_lse:
        lse = None
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = fn(_ptr(xn), _ptr(embed), _ptr(tg), T, D, V, seq, softcap, _ptr(loss), _ptr(lse) if lse is not None else None,
            stream)
    assert rc == 0, lib.ane_op_last_error()
    torch.cuda.synchronize()
    return loss.cpu().numpy(), (lse.cpu().numpy() if lse is not None else None)


def test_noalloc_equals_allocating_entry_twice():
    torch = pytest.importorskip("torch")
    lib = _lib.load()
    big = _case(torch, 8192, 256, 0, 1)      # the bench's 8192 tokens, 256-row blocks
    small = _case(torch, 512, 128, 1, 2)     # then a smaller one (128-row blocks, softcap)
    out_big, out_small = _outputs(torch, big), _outputs(torch, small)
    # the process's first launch from the library loads its code object
    # (kernels and the static scratch) -- HIP's one-time module load, not an
    # allocation of the entry point; a small call does it before measuring
    warm = _case(torch, 128, 64, 0, 3)
    _run(lib, torch, lib.ane_head_loss_noalloc, warm, _outputs(torch, warm))
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    got = [_run(lib, torch, lib.ane_head_loss_noalloc, c, o) for c, o in ((big, out_big), (small, out_small))]
    # without the lse output the scratch holds it; a third call, the big case again
    l3, _ = _run(lib, torch, lib.ane_head_loss_noalloc, big, out_big, with_lse=False)
    free1 = torch.cuda.mem_get_info()[0]
    want = [_run(lib, torch, lib.ane_head_loss, c, o) for c, o in ((big, out_big), (small, out_small))]
    for (gl, gs), (wl, ws) in zip(got, want):
        np.testing.assert_array_equal(gl, wl)
        np.testing.assert_array_equal(gs, ws)
        assert np.isfinite(gl).all() and np.isfinite(gs).all()
    np.testing.assert_array_equal(l3, want[0][0])
    assert free1 == free0   # no device allocation by the three calls


def test_noalloc_refuses_sizes_past_its_scratch():
    torch = pytest.importorskip("torch")
    lib = _lib.load()
    buf = torch.zeros(64, dtype=torch.float32, device="cuda")
    p = _ptr(buf)
    # 16384 tokens of a 32000 vocabulary need ~16 MiB of partials
    rc = lib.ane_head_loss_noalloc(p, p, p, 16384, 768, 32000, 256, 0, p, None, None)
    assert rc == _lib.ANE_ERR_ARG
    msg = lib.ane_op_last_error().decode()
    assert "needs" in msg and "bytes of scratch" in msg and "ntok=16384" in msg
