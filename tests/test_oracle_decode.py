"""Pins the decode oracle (oracle/refdecode.c) on the CPU.

Token-by-token evaluation with a key/value cache must equal one full causal
forward pass: checked against the independent float64 PyTorch model with
grouped-query attention (tests/torch_ref.gqa_logits), against the pinned
full-window oracle (orc_forward_loss) when kv_heads == heads, and for the
greedy rule (first index of the maximum) on its own outputs.
"""
import numpy as np
import torch

import ane
import oracle
import torch_ref


def _params(cfg, seed, std=0.08):
    return ane.init_params(cfg, seed=seed, std=std)


def test_dec_param_count_matches_layout():
    for cfg in (ane.tiny_decode(), ane.decode_gqa(), ane.tiny_decode(kv_heads=4), ane.tiny_decode(kv_heads=1)):
        assert oracle.dec_param_count(cfg) == ane.param_count(cfg)
    # stories110M-shaped blocks with 4 kv heads: 2 * 12 * 768 * 512 fewer weights
    assert ane.param_count(ane.decode_gqa()) == ane.param_count(ane.stories110m("llama2")) - 12 * 2 * 768 * 512


def test_decode_matches_full_forward_gqa():
    cfg = ane.tiny_decode(dim=128, hidden=192, heads=2, kv_heads=1, vocab=96, layers=2)
    p = _params(cfg, 3)
    r = np.random.default_rng(4)
    nseq, plen, nsteps = 2, 9, 5
    prefix = r.integers(0, cfg.vocab, (nseq, plen)).astype(np.uint16)
    forced = r.integers(0, cfg.vocab, (nseq, nsteps)).astype(np.uint16)
    toks, lg = oracle.decode(cfg, p, prefix, nsteps, forced=forced, want_logits=True)
    full = np.concatenate([prefix, forced], 1).astype(np.int64)
    P = torch_ref.params_to_torch(cfg, p, requires_grad=False)
    ref = torch_ref.gqa_logits(cfg, P, torch.tensor(full)).numpy()[:, plen - 1:plen + nsteps]
    np.testing.assert_allclose(lg, ref, atol=2e-4)
    np.testing.assert_array_equal(toks, lg.argmax(-1))


def test_decode_equals_window_oracle_without_grouping():
    cfg = ane.tiny(arch="llama2", vocab=128, seq=16)
    p = _params(cfg, 5)
    r = np.random.default_rng(6)
    seqs = r.integers(0, cfg.vocab, (2, cfg.seq)).astype(np.uint16)
    _, _, full = oracle.forward_loss(cfg, p, seqs, seqs, want_logits=True)  # [n, V, S]
    plen = 10
    toks, lg = oracle.decode(cfg, p, seqs[:, :plen], cfg.seq - plen, forced=seqs[:, plen:], want_logits=True)
    np.testing.assert_allclose(lg[:, :-1], full.transpose(0, 2, 1)[:, plen - 1:cfg.seq - 1], atol=1e-5)


def test_greedy_feeds_back_its_argmax():
    cfg = ane.tiny_decode(vocab=64, layers=1)
    p = _params(cfg, 7, std=0.3)
    prefix = np.random.default_rng(8).integers(0, cfg.vocab, (3, 5)).astype(np.uint16)
    toks, lg = oracle.decode(cfg, p, prefix, 6, want_logits=True)
    toks2, lg2 = oracle.decode(cfg, p, prefix, 6, forced=toks[:, :-1], want_logits=True)
    np.testing.assert_array_equal(toks, toks2)
    np.testing.assert_array_equal(lg, lg2)
    # first index of the maximum on ties
    assert all(int(toks[b, i]) == int(np.flatnonzero(lg[b, i] == lg[b, i].max())[0])
               for b in range(3) for i in range(7))
