"""Evaluation harness: token files, validation loss and bits per byte
(the reference's harness.go:17-89).

``EvalLoss`` keeps the reference's windowing -- the last 10,000 tokens,
windows of 256 at stride 255, the 255 next-token predictions of each window
-- and evaluates all windows in one batched device call.  The reference's
own loop reads the vocab-major logits of ``EvalLogits`` as if they were
position-major (harness.go:63-65; logits are ``logits[v*seq + t]``,
ane/stories/cpu.go:303-327), so its number is not a cross-entropy;
``ReferenceEvalLoss`` reproduces that computation exactly for comparisons
with numbers the reference printed.
"""
from __future__ import annotations

import math

import numpy as np

EVAL_TOKENS = 10_000        # harness.go:35
EVAL_SEQ_LEN = 256          # harness.go:36
AVG_BYTES_PER_TOKEN = 3.7   # harness.go:42


def LoadTokens(path: str) -> np.ndarray:
    """harness.go:17-31: uint16 little-endian token ids."""
    with open(path, "rb") as f:
        data = f.read()
    if len(data) % 2:
        raise ValueError(f"read tokens: file size {len(data)} is not even")
    return np.frombuffer(data, dtype="<u2").astype(np.uint16)


def eval_windows(tokens, eval_tokens: int = EVAL_TOKENS, seq: int = EVAL_SEQ_LEN):
    """Window start offsets into the validation tail (harness.go:53-56)."""
    tokens = np.asarray(tokens)
    if len(tokens) < eval_tokens + seq:
        raise ValueError(f"eval: need at least {eval_tokens + seq} tokens, got {len(tokens)}")
    val = tokens[len(tokens) - eval_tokens:]
    starts = list(range(0, len(val) - seq, seq - 1))
    return val, starts


def EvalLoss(engine, tokens, eval_tokens: int = EVAL_TOKENS) -> float:
    """Mean next-token cross-entropy (nats) over the validation windows,
    batched on the device; the last position of each window has no target
    inside the window and is excluded, as in the reference."""
    seq = engine.cfg.seq
    val, starts = eval_windows(tokens, eval_tokens, seq)
    if not starts:
        raise ValueError("eval: no positions evaluated")
    tok = np.stack([val[p:p + seq] for p in starts]).astype(np.uint16)
    tgt = np.full_like(tok, 0xFFFF)  # ids >= vocab are excluded from the loss
    tgt[:, :-1] = tok[:, 1:]
    per = []
    for i in range(0, len(starts), engine.max_batch):
        _, ps = engine.EvalLoss(tok[i:i + engine.max_batch], tgt[i:i + engine.max_batch])
        per.append(ps)
    # every window contributes seq-1 positions: the mean of window means
    return float(np.mean(np.concatenate(per).astype(np.float64)))


def ValBPB(loss_nats: float) -> float:
    """bits per byte = loss / ln 2 / 3.7 (harness.go:38-42)."""
    return loss_nats / math.log(2) / AVG_BYTES_PER_TOKEN


def ReferenceEvalLoss(engine, tokens, eval_tokens: int = EVAL_TOKENS) -> float:
    """harness.go:46-89 as written: per window, EvalLogits, then rows
    logits[i*V:(i+1)*V] of the vocab-major array taken as position i, the
    running max initialised to the smallest positive float64."""
    seq = engine.cfg.seq
    val, starts = eval_windows(tokens, eval_tokens, seq)
    total, count = 0.0, 0
    for p in starts:
        window = val[p:p + seq]
        logits = engine.EvalLogits(window).astype(np.float64)
        vocab = len(logits) // seq
        for i in range(seq - 1):
            row = logits[i * vocab:(i + 1) * vocab]
            mx = max(float(np.max(row)), 5e-324)
            lse = mx + math.log(float(np.sum(np.exp(row - mx))))
            total -= float(row[int(window[i + 1])]) - lse
            count += 1
    if count == 0:
        raise ValueError("eval: no positions evaluated")
    return total / count
