"""Host-side checks of the per-object seam that make no device call: shape
and weight validation in the C-ABI (refused before any HIP call), the
reference's length checks (checkLen, ane/backward_darwin.go:397-402), nil
objects, and newOffload's nil result when the accelerator is off
(ane/offload_darwin.go:81-89)."""
import numpy as np
import pytest

from ane import objects


def weights(dim, hidden):
    z = lambda o, i: np.zeros((o, i), np.float32)
    return {"wq": z(dim, dim), "wk": z(dim, dim), "wv": z(dim, dim), "wo": z(dim, dim), "w1": z(hidden, dim),
            "w2": z(dim, hidden)}


@pytest.mark.parametrize("dim,hidden,heads,seq,msg", [
    (128, 256, 3, 64, "dim=128 hidden=256 heads=3 seq=64"),
    (128, 200, 2, 64, "hidden=200"),
    (128, 256, 2, 96, "seq=96"),
    (128, 256, 2, 576, "seq=576"),
])
def test_layer_forward_refuses_shapes(dim, hidden, heads, seq, msg):
    with pytest.raises(objects.SeamError, match=f"compile layer forward: invalid shape .*{msg}"):
        objects.compile_stories_layer_forward(weights(dim, hidden), seq, heads=heads)


def test_layer_backward_refuses_long_sequences():
    with pytest.raises(objects.SeamError, match="compile layer backward: invalid shape .*seq=320"):
        objects.compile_stories_layer_backward(weights(128, 256), 320, heads=2)


def test_weight_lengths_are_checked():
    w = weights(128, 256)
    w["w2"] = np.zeros((128, 255), np.float32)
    with pytest.raises(objects.SeamError, match="compile layer forward: w2 len=32640 want=32768"):
        objects.compile_stories_layer_forward(w, 64, heads=2)


def test_buffer_lengths_and_nil_objects():
    lf = objects.LayerForward(None, 128, 256, 2, 64)
    with pytest.raises(objects.SeamError, match="run layer forward: input len=100 want=8192"):
        lf.run(np.zeros(8192, np.float32), np.zeros(100, np.float32))
    with pytest.raises(objects.SeamError, match="run layer forward: layer is nil"):
        lf.run(np.zeros(8192, np.float32), np.zeros(8192, np.float32))
    lb = objects.LayerBackward(None, 128, 256, 2, 64)
    n = 128 * 64
    with pytest.raises(objects.SeamError, match="run layer backward attention: dx2 len=5 want=8192"):
        lb.run_attention(*[np.zeros(n, np.float32)] * 7, np.zeros(5, np.float32))
    with pytest.raises(objects.SeamError, match="run layer backward ffn: h1 len=8192 want=16384"):
        lb.run_ffn(np.zeros(n, np.float32), np.zeros(2 * n, np.float32), np.zeros(n, np.float32),
                   np.zeros(n, np.float32))
    with pytest.raises(objects.SeamError, match="must be a C-contiguous float32 array"):
        lb.run_ffn(np.zeros(n, np.float64), np.zeros(2 * n, np.float32), np.zeros(n, np.float32),
                   np.zeros(2 * n, np.float32))


def test_offload_off_and_refused_shapes():
    embed = np.zeros((1024, 128), np.float32)
    assert objects.new_offload(embed, 64, use_ane=False) is None
    assert objects.refresh_offload(None, embed, 64, use_ane=False) is None
    with pytest.raises(objects.SeamError, match="new offload: invalid shape vocab=1000"):
        objects.new_offload(np.zeros((1000, 128), np.float32), 64)
    off = objects.Offload(None, 1024, 128, 64)
    assert not (off.has_rms_forward() or off.has_classifier_forward() or off.has_softmax())
    with pytest.raises(objects.SeamError, match="run rms forward: offload is nil"):
        off.run_rms_forward(np.zeros(128 * 64, np.float32), np.zeros(128 * 64, np.float32))
