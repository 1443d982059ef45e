"""Layers without rotary positions (NoPE: TDecoderLayerSpec.NoRope,
src/infer/mormot.ai.infer.decoder.pas:139; SmolLM3's no_rope_layers,
src/infer/mormot.ai.infer.model.qwen3.pas:28-33) in the oracle, pinned by
what the mathematics fixes:

- at position 0 the rotation angle is 0 (cos 1, sin 0), so a one-token
  forward of a model whose layers are all NoPE equals the same model with
  rotary positions, bit for bit;
- with more tokens the two differ (the flag takes effect);
- one NoPE layer over embeddings: the last token's keys and values of the
  earlier tokens depend on those tokens alone and nothing carries their
  order, so its logits are the same for any order of the earlier tokens (up
  to the order of the softmax sums); with rotary positions they are not.

The device against this oracle: test_gpu_model.py (the NoPE rows of TINY)."""
import numpy as np

import oracle_lib as O
from infer_hip import models

SHAPE = dict(layers=2, vocab=512, hidden=128, heads=4, kv_heads=2, head_dim=32, ffn=256,
             qk_norm=False)


def logits(over, ids, seed=5):
    spec = models.Spec(models.tiny("qwen3-0.6b-q8_0", **{**SHAPE, **over}), seed=seed)
    m = O.Model(spec, 32)
    y = m.forward(np.array(ids, np.int32))
    m.close()
    return y


def test_nope_at_position_0_is_rope():
    a = logits(dict(no_rope_interval=1), [7])
    b = logits({}, [7])
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_nope_differs_after_position_0():
    a = logits(dict(no_rope_interval=1), [7, 300, 41, 9])
    b = logits({}, [7, 300, 41, 9])
    assert np.abs(a - b).max() > 1e-4 * np.abs(b).max()


def test_nope_one_layer_order_of_earlier_tokens():
    nope = dict(layers=1, no_rope_interval=1)
    a = logits(nope, [7, 300, 41, 9])
    b = logits(nope, [41, 7, 300, 9])
    assert np.abs(a - b).max() <= 1e-5 * np.abs(a).max()
    r = logits(dict(layers=1), [7, 300, 41, 9])
    s = logits(dict(layers=1), [41, 7, 300, 9])
    assert np.abs(r - s).max() > 1e-4 * np.abs(r).max()


def test_nope_interval_marks_layers():
    spec = models.Spec(models.tiny("qwen3-0.6b-q8_0", **{**SHAPE, "layers": 4, "no_rope_interval": 2}))
    flags = [spec.struct.layer[i].no_rope for i in range(4)]
    assert flags == [0, 1, 0, 1]
