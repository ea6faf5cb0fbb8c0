"""Greedy KV-cache decoding on the GPU against the CPU decode oracle
(oracle/refdecode.c, pinned in tests/test_oracle_decode.py).

The per-layer GEMM chain has three implementations -- one fused launch per
layer whose consumers poll the exchanged data itself (the default where every
block of it fits on the GPU at once), the same launch with done counters
(ANE_DEC_TAIL=1), and one launch per GEMM (ANE_DEC_TAIL=0) -- and the
model-level tests run all three.

Logits are compared at max-abs <= 2e-2 (fp16 weights, activations and KV
cache; fp32 accumulation), the contract's logit tolerance.  Greedy choices
are checked the way a tolerance allows: the token the GPU picks must have an
oracle logit within 2e-2 of the oracle's maximum (an exact tie-break between
logits closer than the tolerance is not a parity statement).
"""
import numpy as np
import pytest

import ane
import oracle
from ane import _lib

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _setup(cfg, nseq, plen, seed, std=0.05):
    p = ane.init_params(cfg, seed=seed, std=std)
    r = np.random.default_rng(seed + 1)
    prefix = r.integers(0, cfg.vocab, (nseq, plen)).astype(np.uint16)
    return p, prefix


def _check_choice(gpu_tok, ref_logits):
    top = ref_logits.max(-1)
    picked = np.take_along_axis(ref_logits, gpu_tok[..., None].astype(np.int64), -1)[..., 0]
    assert np.all(picked >= top - TOL), (picked - top).min()


def test_prefill_and_forced_steps_match_oracle():
    cfg = ane.tiny_decode()
    nseq, plen, nsteps = 3, 128, 6
    p, prefix = _setup(cfg, nseq, plen, 11)
    forced = np.random.default_rng(12).integers(0, cfg.vocab, (nseq, nsteps)).astype(np.uint16)
    ref_tok, ref_lg = oracle.decode(cfg, p, prefix, nsteps, forced=forced, want_logits=True)
    dec = ane.Decoder(cfg, p, max_batch=4, max_ctx=256)
    try:
        t0, lg0 = dec.Prefill(prefix, want_logits=True)
        errs = [np.abs(lg0 - ref_lg[:, 0]).max()]
        _check_choice(t0, ref_lg[:, 0])
        np.testing.assert_array_equal(t0, lg0.argmax(-1))
        for i in range(nsteps):
            ti, lgi = dec.Step(forced[:, i], want_logits=True)
            errs.append(np.abs(lgi - ref_lg[:, i + 1]).max())
            _check_choice(ti, ref_lg[:, i + 1])
        assert dec.Position() == plen + nsteps
    finally:
        dec.Close()
    print("decode logits max-abs err per step", [f"{e:.2e}" for e in errs])
    assert max(errs) <= TOL


@pytest.mark.parametrize("form", ["split", "wide"])
@pytest.mark.parametrize("heads,kv_heads", [(4, 4), (4, 1), (6, 2)])
def test_query_head_groups(heads, kv_heads, form, monkeypatch):
    """Every head-group size the attention kernels are built for (1, 4, 3
    query heads per key/value head), in both decode-attention forms, through
    prefill and forced steps, with hidden 256 and dim 64 * heads (K of 1, 4
    and 6 windows per split-K GEMM) and a context that crosses a 256-key
    split."""
    monkeypatch.setenv("ANE_DEC_ATTN", form)
    cfg = ane.tiny_decode(heads=heads, kv_heads=kv_heads, dim=64 * heads, hidden=256, layers=1)
    nseq, plen, nsteps = 2, 320, 3
    p, prefix = _setup(cfg, nseq, plen, 41)
    forced = np.random.default_rng(42).integers(0, cfg.vocab, (nseq, nsteps)).astype(np.uint16)
    ref_tok, ref_lg = oracle.decode(cfg, p, prefix, nsteps, forced=forced, want_logits=True)
    dec = ane.Decoder(cfg, p, max_batch=2, max_ctx=384)
    try:
        t0, lg0 = dec.Prefill(prefix, want_logits=True)
        errs = [np.abs(lg0 - ref_lg[:, 0]).max()]
        for i in range(nsteps):
            ti, lgi = dec.Step(forced[:, i], want_logits=True)
            errs.append(np.abs(lgi - ref_lg[:, i + 1]).max())
            _check_choice(ti, ref_lg[:, i + 1])
    finally:
        dec.Close()
    print(f"G={heads // kv_heads} decode logits max-abs err per step", [f"{e:.2e}" for e in errs])
    assert max(errs) <= TOL


@pytest.mark.parametrize("form", ["split", "wide"])
@pytest.mark.parametrize("plen,max_ctx", [(64, 128), (256, 512)])
def test_cache_positions_never_read_before_written(plen, max_ctx, form, monkeypatch):
    """The KV cache starts as NaN bit patterns: prefill, every decode step
    (whose new k/v row is formed and used inside the attention kernel) and
    the key splits past the context must never let a stale row reach the
    logits -- a NaN anywhere would show."""
    monkeypatch.setenv("ANE_DEC_ATTN", form)
    cfg = ane.tiny_decode()
    nseq, nsteps = 2, 3
    p, prefix = _setup(cfg, nseq, plen, 71)
    forced = np.random.default_rng(72).integers(0, cfg.vocab, (nseq, nsteps)).astype(np.uint16)
    ref_tok, ref_lg = oracle.decode(cfg, p, prefix, nsteps, forced=forced, want_logits=True)
    dec = ane.Decoder(cfg, p, max_batch=2, max_ctx=max_ctx)
    try:
        dec.DebugFillCache(0xFF)
        _, lg0 = dec.Prefill(prefix, want_logits=True)
        lgs = [lg0] + [dec.Step(forced[:, i], want_logits=True)[1] for i in range(nsteps)]
    finally:
        dec.Close()
    lg = np.stack(lgs, 1)
    assert np.isfinite(lg).all()
    assert np.abs(lg - ref_lg).max() <= TOL


@pytest.mark.parametrize("form", ["split", "wide"])
@pytest.mark.parametrize("plen,max_ctx", [(1024, 1152), (1280, 2304)])
def test_long_prefix_multi_chunk_attention(form, plen, max_ctx, monkeypatch):
    """Long prefixes: prefill attention streams 8-10 key chunks.  Decode
    attention in both forms: 256-thread blocks over 5 or 9 context splits,
    and 1024-thread blocks holding up to 1152 keys (one split written
    directly, or two merged; the bench batch picks this form by itself)."""
    monkeypatch.setenv("ANE_DEC_ATTN", form)
    cfg = ane.tiny_decode(layers=1)
    nseq, nsteps = 2, 3
    p, prefix = _setup(cfg, nseq, plen, 21)
    forced = np.random.default_rng(22).integers(0, cfg.vocab, (nseq, nsteps)).astype(np.uint16)
    ref_tok, ref_lg = oracle.decode(cfg, p, prefix, nsteps, forced=forced, want_logits=True)
    dec = ane.Decoder(cfg, p, max_batch=2, max_ctx=max_ctx)
    try:
        _, lg0 = dec.Prefill(prefix, want_logits=True)
        errs = [np.abs(lg0 - ref_lg[:, 0]).max()]
        for i in range(nsteps):
            _, lgi = dec.Step(forced[:, i], want_logits=True)
            errs.append(np.abs(lgi - ref_lg[:, i + 1]).max())
    finally:
        dec.Close()
    print("long-prefix logits max-abs err", [f"{e:.2e}" for e in errs])
    assert max(errs) <= TOL


@pytest.mark.parametrize("tail", ["2", "1", "0"])
def test_generate_graph_equals_eager_steps_and_oracle_choices(tail, monkeypatch):
    monkeypatch.setenv("ANE_DEC_TAIL", tail)
    cfg = ane.tiny_decode()
    nseq, plen, nsteps = 4, 64, 12
    p, prefix = _setup(cfg, nseq, plen, 31, std=0.08)
    dec = ane.Decoder(cfg, p, max_batch=8, max_ctx=128)
    try:
        t0, _ = dec.Prefill(prefix)
        gen = dec.Generate(nsteps)
        assert gen.shape == (nseq, nsteps)
        assert dec.Position() == plen + nsteps
        dec.Prefill(prefix)
        eager = np.stack([dec.Step()[0] for _ in range(nsteps)], 1)
        # a second Generate call replays the same graph from the new position
        more = dec.Generate(3)
    finally:
        dec.Close()
    np.testing.assert_array_equal(gen, eager)
    assert more.shape == (nseq, 3)
    # every greedy choice is (to tolerance) the oracle's argmax given the same history
    inputs = np.concatenate([t0[:, None], gen[:, :-1]], 1)
    _, ref_lg = oracle.decode(cfg, p, prefix, nsteps, forced=inputs, want_logits=True)
    _check_choice(t0, ref_lg[:, 0])
    _check_choice(gen, ref_lg[:, 1:])


@pytest.mark.parametrize("tail", ["2", "1", "0"])
@pytest.mark.parametrize("form", ["split", "wide"])
def test_full_size_gqa_model_matches_oracle(form, tail, monkeypatch):
    """The decode benchmark's model (12 layers, dim 768, 12/4 heads,
    vocab 32000), two sequences, 64-token prefix, three forced steps, in
    both decode-attention forms and both GEMM-chain forms."""
    monkeypatch.setenv("ANE_DEC_ATTN", form)
    monkeypatch.setenv("ANE_DEC_TAIL", tail)
    cfg = ane.decode_gqa()
    nseq, plen, nsteps = 2, 64, 3
    p, prefix = _setup(cfg, nseq, plen, 4, std=0.02)
    forced = np.random.default_rng(41).integers(0, cfg.vocab, (nseq, nsteps)).astype(np.uint16)
    _, ref_lg = oracle.decode(cfg, p, prefix, nsteps, forced=forced, want_logits=True)
    dec = ane.Decoder(cfg, p, max_batch=64, max_ctx=1152)
    try:
        _, lg0 = dec.Prefill(prefix, want_logits=True)
        errs = [np.abs(lg0 - ref_lg[:, 0]).max()]
        for i in range(nsteps):
            _, lgi = dec.Step(forced[:, i], want_logits=True)
            errs.append(np.abs(lgi - ref_lg[:, i + 1]).max())
    finally:
        dec.Close()
    print("full-size decode logits max-abs err", [f"{e:.2e}" for e in errs])
    assert max(errs) <= TOL


def test_decoder_errors():
    cfg = ane.tiny_decode()
    p, prefix = _setup(cfg, 2, 64, 51)
    with pytest.raises(ane.EngineError) as ei:
        ane.Decoder(cfg, p, max_batch=65)
    assert ei.value.code == _lib.ANE_ERR_ARG
    dec = ane.Decoder(cfg, p, max_batch=2, max_ctx=128)
    try:
        with pytest.raises(ane.EngineError) as ei:
            dec.Step()
        assert ei.value.code == _lib.ANE_ERR_STATE
        with pytest.raises(ane.EngineError) as ei:
            dec.Prefill(prefix[:, :40])
        assert ei.value.code == _lib.ANE_ERR_ARG and "multiple of 64" in str(ei.value)
        with pytest.raises(ane.EngineError):
            dec.Prefill(np.zeros((3, 64), np.uint16))
        dec.Prefill(prefix)
        with pytest.raises(ane.EngineError) as ei:
            dec.Generate(65)
        assert ei.value.code == _lib.ANE_ERR_ARG
        with pytest.raises(ane.EngineError):
            dec.SetParams(p[:-1])
    finally:
        dec.Close()
    with pytest.raises(ane.EngineError) as ei:
        dec.Step()
    assert ei.value.code == _lib.ANE_ERR_CLOSED


@pytest.mark.parametrize("tail", ["2", "1", "0"])
@pytest.mark.parametrize("heads,kv_heads", [(4, 2), (6, 2), (3, 1)])
def test_full_batch_of_64_every_sequence(heads, kv_heads, tail, monkeypatch):
    """64 sequences (every decode row) at dims 256, 384 and 192: the
    classifier splits K over 2, 3 and 2 waves (4, 6 and 3 windows; one wave
    holding a single zeroed-surplus window at 192), and the argmax transpose
    covers tokens 62-63 of the last MFMA tile.  Prefill, forced steps, and
    greedy Generate, every sequence against the oracle."""
    monkeypatch.setenv("ANE_DEC_TAIL", tail)
    cfg = ane.tiny_decode(heads=heads, kv_heads=kv_heads, dim=64 * heads, layers=1)
    nseq, plen, nsteps = 64, 64, 2
    p, prefix = _setup(cfg, nseq, plen, 81)
    forced = np.random.default_rng(82).integers(0, cfg.vocab, (nseq, nsteps)).astype(np.uint16)
    ref_tok, ref_lg = oracle.decode(cfg, p, prefix, nsteps, forced=forced, want_logits=True)
    dec = ane.Decoder(cfg, p, max_batch=64, max_ctx=128)
    try:
        t0, lg0 = dec.Prefill(prefix, want_logits=True)
        errs = [np.abs(lg0 - ref_lg[:, 0]).max()]
        _check_choice(t0, ref_lg[:, 0])
        np.testing.assert_array_equal(t0, lg0.argmax(-1))
        for i in range(nsteps):
            ti, lgi = dec.Step(forced[:, i], want_logits=True)
            errs.append(np.abs(lgi - ref_lg[:, i + 1]).max())
            _check_choice(ti, ref_lg[:, i + 1])
            np.testing.assert_array_equal(ti, lgi.argmax(-1))
        dec.Prefill(prefix)
        gen = dec.Generate(3)
    finally:
        dec.Close()
    print(f"dim {cfg.dim}, 64 sequences: logits max-abs err per step", [f"{e:.2e}" for e in errs])
    assert max(errs) <= TOL
    inputs = np.concatenate([t0[:, None], gen[:, :-1]], 1)
    _, g_lg = oracle.decode(cfg, p, prefix, 3, forced=inputs, want_logits=True)
    _check_choice(gen, g_lg[:, 1:])


@pytest.mark.parametrize("tail,form", [("2", None), ("2", "wide"), ("1", None)])
def test_fused_chain_wait_timeout_falls_back(tail, form, monkeypatch):
    """A dependency wait of the fused layer kernel that times out does not
    fail the call: the decoder switches for good to one launch per GEMM and
    redoes the call from its start (the reference's latch-and-continue,
    ane/engine.go:887-894).  The host forces the timeout (a poll limit of 0
    fails every wait at once, and every block still exits).  The redone
    Step and Generate, and the steps after them, match the oracle: no cache
    row that a failed launch touched is read before the redo rewrites it.
    With the wide attention form forced, the polling chain's launches also
    hold the next layer's attention blocks, whose q wait fails the same way."""
    cfg = ane.tiny_decode()
    nseq, plen = 2, 64
    p, prefix = _setup(cfg, nseq, plen, 61)
    monkeypatch.setenv("ANE_DEC_TAIL", tail)
    if form:
        monkeypatch.setenv("ANE_DEC_ATTN", form)
    monkeypatch.setenv("ANE_DEC_TAIL_SPIN", "0")
    forced = np.random.default_rng(62).integers(0, cfg.vocab, (nseq, 2)).astype(np.uint16)
    _, ref_lg = oracle.decode(cfg, p, prefix, 2, forced=forced, want_logits=True)

    dec = ane.Decoder(cfg, p, max_batch=nseq, max_ctx=128)
    try:
        assert dec.FusedChain() == 1
        _, lg0 = dec.Prefill(prefix, want_logits=True)
        _, lg1 = dec.Step(forced[:, 0], want_logits=True)  # the chain fails; redone per GEMM
        assert dec.FusedChain() == 2
        _, lg2 = dec.Step(forced[:, 1], want_logits=True)
        assert dec.Position() == plen + 2
    finally:
        dec.Close()
    errs = [np.abs(lg - ref_lg[:, i]).max() for i, lg in enumerate((lg0, lg1, lg2))]
    print("logits max-abs err (prefill, redone step, next step)", [f"{e:.2e}" for e in errs])
    assert max(errs) <= TOL

    # the failure inside a replayed step graph: Generate redone with the
    # per-GEMM graph, then continued
    dec = ane.Decoder(cfg, p, max_batch=nseq, max_ctx=128)
    try:
        t0, _ = dec.Prefill(prefix)
        gen = dec.Generate(3)
        assert dec.FusedChain() == 2 and dec.Position() == plen + 3
        gen2 = dec.Generate(2)
    finally:
        dec.Close()
    inputs = np.concatenate([t0[:, None], gen, gen2[:, :-1]], 1)
    _, g_lg = oracle.decode(cfg, p, prefix, 5, forced=inputs, want_logits=True)
    _check_choice(np.concatenate([gen, gen2], 1), g_lg[:, 1:])

    # without the forced timeout a new decoder keeps the chain
    monkeypatch.delenv("ANE_DEC_TAIL_SPIN")
    dec = ane.Decoder(cfg, p, max_batch=nseq, max_ctx=128)
    try:
        dec.Prefill(prefix)
        dec.Step(forced[:, 0])
        assert dec.FusedChain() == 1
    finally:
        dec.Close()
