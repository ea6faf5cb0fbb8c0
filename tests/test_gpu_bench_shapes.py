"""Parity at the exact shapes bench.py reports, against the oracle's values
for the same inputs (committed fixtures written by
tests/golden/make_golden.py --bench; the oracle takes minutes at these
sizes, so it does not run here).

* B32 x 256 forward + loss: the bench's own call,
  EvalLossWindows over the resident stream, which runs the 8-wave 256x256
  W1|W3 and classifier tiles, the 128x192 QKV tile and 256-row CE partials;
  all 32 per-sequence losses within 1e-3 nats.
* B16 x 256 gradients, both architectures: the split-K weight
  gradient GEMMs at K = 4096 tokens and the B16 tile rules; per-segment
  norms and sampled rows at relative L2 <= 1e-2 (the token embedding: the
  whole tensor's error, estimated from a stratified sample of its token and
  other rows).
* B16 nanochat compat on windows that each repeat one id: the scalar
  lambdas' gradients, the smear lambda's included (a sum that nearly cancels
  on random windows), within 1e-2 of the oracle's.
* 64 sequences x 1024-token prefix decode in the attention form
  the batch size selects: prefill and three forced steps, the logits of four
  sampled sequences within 2e-2, and the replayed-graph Generate path's
  greedy tokens against the oracle's.
"""
import numpy as np
import pytest

import ane
from golden_io import BENCH_EMBED_ROWS, embed_row_split, load, repeated_windows, sampled_rows, stratified_rel_l2

pytestmark = pytest.mark.gpu

SCALARS = ("resid_lambdas", "x0_lambdas", "smear_lambda", "backout_lambda", "ve_gate")


def test_bench_forward_b32_every_sequence():
    cfg = ane.stories110m("llama2")
    params = ane.init_params(cfg, seed=0, std=0.02)
    B, S = 32, cfg.seq
    tok, tgt = ane.make_tokens(cfg, B, seed=2)
    # the resident stream and window positions bench.py builds
    stream = np.concatenate([np.concatenate([tok[b], tgt[b][-1:]]) for b in range(B)]).astype(np.uint16)
    pos = np.arange(B, dtype=np.uint64) * np.uint64(S + 1)
    ref, tol = load("bench_fwd_b32_llama2_loss_per_seq")
    eng = ane.Open(ane.Options(Config=cfg, Params=params, MaxBatch=B, Tokens=stream))
    try:
        mean, per = eng.EvalLossWindows(pos)
        mean2, per2 = eng.EvalLossWindows(pos)   # the same call again
        mean3, per3 = eng.EvalLoss(tok, tgt)      # explicit host tokens, same kernels
    finally:
        eng.Destroy()
    err = np.abs(per.astype(np.float64) - ref.astype(np.float64))
    print(f"B32 forward: mean {mean:.6f} oracle {ref.astype(np.float64).mean():.6f}; per-seq max err {err.max():.2e}")
    assert err.max() <= tol
    assert abs(mean - ref.astype(np.float64).mean()) <= tol
    np.testing.assert_array_equal(per2, per)
    np.testing.assert_array_equal(per3, per)


def _rows(cfg, g, tokens):
    out = []
    for i, (name, off, shape) in enumerate(ane.param_layout(cfg)):
        seg = g[off:off + int(np.prod(shape))]
        idx = sampled_rows(cfg, name.split(".")[-1], shape, tokens, 90 + i)
        out.append(seg if idx is None else seg.reshape(shape)[idx].reshape(-1))
    return out


@pytest.mark.parametrize("arch,mode", [("llama2", "true"), ("nanochat", "compat")])
def test_bench_grads_b16(arch, mode):
    cfg = ane.stories110m(arch, grad_mode=mode)
    params = ane.init_params(cfg, seed=0, std=0.02)
    tok, tgt = ane.make_tokens(cfg, 16, seed=3)
    key = f"bench_grads_b16_{arch}_{mode}"
    ref_norms, tol = load(key + "_norms")
    ref_rows, _ = load(key + "_rows")
    ref_loss, ltol = load(key + "_loss")
    eng = ane.Open(ane.Options(Config=cfg, Params=params, MaxBatch=16))
    try:
        loss, g = eng.Grads(tok, tgt)
    finally:
        eng.Destroy()
    assert abs(loss - float(ref_loss[0])) <= ltol
    def bound(name):
        if name == "smear_lambda":
            # one sum over 16 x 256 x 768 products that nearly cancels: its
            # value moves ~10% between builds that differ only in last-bit
            # fp32 rounding (as at B1, test_gpu_train)
            return 0.25
        return 5e-2 if name.split(".")[-1] in SCALARS else tol


    def rel(a, b):
        return np.linalg.norm(a.astype(np.float64) - b) / max(np.linalg.norm(b), 1e-30)

    rows = _rows(cfg, g, tok)
    off = 0
    worst = []
    for (name, seg_off, shape), n_ref, got in zip(ane.param_layout(cfg), ref_norms, rows):
        want = ref_rows[off:off + got.size].astype(np.float64)
        off += got.size
        if name == "embed":
            # The whole tensor's relative L2 error, estimated from the
            # stratified sample: BENCH_EMBED_ROWS of the batch's token rows
            # (classifier part + the back-propagated lookup gradient) and as
            # many of the other rows (classifier part only), each stratum
            # weighted by its row count.  The token rows hold nearly all of
            # the norm, so this is their error.
            tok_rows, other = embed_row_split(shape, tok)
            e_all = stratified_rel_l2(got, want, 2, (len(tok_rows) / BENCH_EMBED_ROWS, len(other) / BENCH_EMBED_ROWS))
            k = got.size // 2
            e_tok, e_oth = rel(got[:k], want[:k]), rel(got[k:], want[k:])
            print(f"embed: whole-tensor estimate {e_all:.3e} (token rows {e_tok:.3e}, other rows {e_oth:.3e})")
            worst += [(e_all, "embed")]
            assert e_all <= tol, (e_all, e_tok, e_oth)
            assert e_oth <= tol, e_oth
        else:
            e_rows = rel(got, want)
            worst.append((e_rows, name))
            assert e_rows <= bound(name), (name, e_rows)
        n_got = np.linalg.norm(g[seg_off:seg_off + int(np.prod(shape))].astype(np.float64))
        assert abs(n_got - n_ref) <= bound(name) * max(n_ref, 1e-30), (name, n_got, n_ref)
    assert off == ref_rows.size
    worst.sort(reverse=True)
    print(f"B16 {arch}/{mode}: loss {loss:.6f} oracle {float(ref_loss[0]):.6f}; worst sampled-row rel L2 "
          f"{[(n, f'{e:.2e}') for e, n in worst[:4]]}")


def test_bench_smear_lambda_well_conditioned():
    """nanochat compat at B16 (full size) on windows that each repeat one
    id: the smear lambda's gradient (ane/common.go:343-382) is then a sum
    that does not cancel (rounding only the parameters to fp16 moves the
    oracle's value by 3e-4, against ~17% on random windows), so the device
    value is held to the weight-gradient bound 1e-2 against the oracle's
    (measured 3.5e-5); the other scalar lambdas alike."""
    cfg = ane.stories110m("nanochat", grad_mode="compat")
    params = ane.init_params(cfg, seed=0, std=0.02)
    tok, tgt = repeated_windows(cfg, 16, 5)
    ref, tol = load("bench_grads_b16_nanochat_compat_repeat_scalars")
    ref_loss, ltol = load("bench_grads_b16_nanochat_compat_repeat_loss")
    eng = ane.Open(ane.Options(Config=cfg, Params=params, MaxBatch=16))
    try:
        loss, g = eng.Grads(tok, tgt)
    finally:
        eng.Destroy()
    assert abs(loss - float(ref_loss[0])) <= ltol
    off = 0
    for name, seg_off, shape in ane.param_layout(cfg):
        if name not in ("resid_lambdas", "x0_lambdas", "smear_lambda", "backout_lambda"):
            continue
        n = int(np.prod(shape))
        got, want = g[seg_off:seg_off + n].astype(np.float64), ref[off:off + n].astype(np.float64)
        off += n
        err = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
        print(f"{name}: device {got[:3]} oracle {want[:3]} rel L2 {err:.2e}")
        assert err <= tol, (name, err)
    assert off == ref.size


@pytest.mark.parametrize("tail", ["2", "1", "0"])
def test_bench_decode_b64_prefix1024(tail, monkeypatch):
    monkeypatch.setenv("ANE_DEC_TAIL", tail)  # the chain polling its data (the bench's), with done counters, one launch per GEMM
    cfg = ane.decode_gqa()
    params = ane.init_params(cfg, seed=4, std=0.02)
    batch, plen, steps = 64, 1024, 3
    prefix = np.random.default_rng(4).integers(0, cfg.vocab, (batch, plen)).astype(np.uint16)
    sel, _ = load("bench_decode_b64_seqs")
    sel = sel.astype(np.int64)
    ref_tok, _ = load("bench_decode_b64_tokens")   # [4, steps + 1]
    ref_lg, tol = load("bench_decode_b64_logits")  # [4, steps + 1, V] fp16
    ref_lg = ref_lg.astype(np.float32)
    dec = ane.Decoder(cfg, params, max_batch=batch, max_ctx=plen + 128)  # the bench's decoder
    try:
        t0, lg0 = dec.Prefill(prefix, want_logits=True)
        errs = [np.abs(lg0[sel] - ref_lg[:, 0]).max()]
        prev = t0.copy()
        for i in range(steps):
            forced = prev.copy()
            forced[sel] = ref_tok[:, i]         # the oracle's greedy history for the sampled sequences
            ti, lgi = dec.Step(forced, want_logits=True)
            errs.append(np.abs(lgi[sel] - ref_lg[:, i + 1]).max())
            prev = ti
        # the bench's path: prefill again, then greedy steps from the replayed graph
        g0, _ = dec.Prefill(prefix)
        gen = dec.Generate(steps)
    finally:
        dec.Close()
    print("B64 decode logits max-abs err per position", [f"{e:.2e}" for e in errs])
    assert max(errs) <= tol
    np.testing.assert_array_equal(g0, t0)
    # greedy choices: while the device's history equals the oracle's, each
    # token must be (to the logit tolerance) the oracle's argmax
    got = np.concatenate([g0[sel, None], gen[sel]], 1)   # [4, steps + 1]
    agree = 0
    for s in range(len(sel)):
        for i in range(steps + 1):
            top = ref_lg[s, i].max()
            assert ref_lg[s, i, got[s, i]] >= top - tol, (s, i)
            if got[s, i] != ref_tok[s, i]:
                break          # a near-tie took another branch; later positions have another history
            agree += 1
    print(f"greedy tokens equal to the oracle's: {agree} of {len(sel) * (steps + 1)}")
