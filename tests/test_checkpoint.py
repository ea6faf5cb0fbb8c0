"""V5 checkpoint + SANE trailer format (ane/checkpoint.py) on the CPU: the
size formula against storiesCheckpointSize (ane/engine.go:769-791) restated
by hand for the reference's model, the header bytes, the section order and
a write/read round trip."""
import struct

import numpy as np
import pytest

import ane
from ane.checkpoint import TrainMeta, checkpoint_size, read_checkpoint, write_checkpoint


def test_size_matches_reference_formula():
    cfg = ane.stories110m("nanochat")
    D, H, V, L = 768, 2048, 32000, 12
    wq = D * D
    layer_w = L * (wq * 3 + wq + H * D + D * H)
    layer_o = L * (wq * 6 + wq * 2 + H * D * 2 + D * H * 2)
    ve_layers = [l for l in range(L) if ane.is_ve_layer(cfg, l)]
    assert len(ve_layers) == 6
    layer_w += len(ve_layers) * (V * D + 12 * 12)
    layer_o += len(ve_layers) * (2 * V * D + 2 * 12 * 12)
    model = V * D * 3 + L * 3 + L * 3 + D * D * 3 + 3 + 3
    assert checkpoint_size(cfg) == 96 + 4 * (layer_w + layer_o + model)


def test_llama2_has_no_v5_layout(tmp_path):
    with pytest.raises(ValueError, match="nanochat model only"):
        checkpoint_size(ane.stories110m("llama2"))


def test_round_trip_and_layout(tmp_path):
    cfg = ane.tiny("nanochat", layers=3)
    n = ane.param_count(cfg)
    r = np.random.default_rng(0)
    p, m, v, g = (r.standard_normal(n).astype(np.float32) for _ in range(4))
    meta = TrainMeta(Step=7, TotalSteps=100, LR=float(np.float32(3e-4)), Loss=2.5, CumCompile=1.0, CumTrain=12.5, CumWall=20.0,
                     CumSteps=7, CumBatches=3, AdamT=3)
    path = str(tmp_path / "ck" / "model.bin")
    write_checkpoint(path, cfg, meta, p, m, v, token_pos=1234, pending=2, accum=g)
    raw = open(path, "rb").read()
    size = checkpoint_size(cfg)
    assert len(raw) == size + 4 + 16 + 4 * n
    hdr = struct.unpack("<10i2f3d3i3i", raw[:96])
    assert hdr[:10] == (0x424C5A54, 5, 7, 100, cfg.layers, cfg.vocab, cfg.dim, cfg.hidden, cfg.heads, cfg.seq)
    assert hdr[15:18] == (7, 3, 3) and hdr[18:] == (0, 0, 0)
    # section order: the first layer's Wq follows the header; its Adam M
    # follows the last layer's weights; the embedding is followed by its M, V
    lay = ane.param_layout(cfg)
    wq0 = np.frombuffer(raw[96:96 + 4 * cfg.dim * cfg.dim], "<f4")
    np.testing.assert_array_equal(wq0, p[:cfg.dim * cfg.dim])
    layers_end = max(off + int(np.prod(s)) for name, off, s in lay if name.startswith("layers."))
    m0 = np.frombuffer(raw[96 + 4 * layers_end:96 + 4 * layers_end + 16], "<f4")
    np.testing.assert_array_equal(m0, m[:4])
    assert raw[size:size + 4] == b"SANE"
    assert struct.unpack("<IQI", raw[size + 4:size + 20]) == (2, 1234, 2)
    meta2, p2, m2, v2, tr = read_checkpoint(path, cfg)
    assert meta2 == meta
    for a, b in ((p, p2), (m, m2), (v, v2), (g, tr["accum"])):
        np.testing.assert_array_equal(a, b)
    assert tr["token_pos"] == 1234 and tr["pending"] == 2


def test_rejects_other_configs(tmp_path):
    cfg = ane.tiny("nanochat")
    n = ane.param_count(cfg)
    z = np.zeros(n, np.float32)
    path = str(tmp_path / "a.bin")
    write_checkpoint(path, cfg, TrainMeta(), z, z, z)
    with pytest.raises(ValueError, match="config mismatch"):
        read_checkpoint(path, ane.tiny("nanochat", layers=4))
    open(path, "r+b").write(struct.pack("<i", 0x1234))
    with pytest.raises(ValueError, match="bad checkpoint header"):
        read_checkpoint(path, cfg)
