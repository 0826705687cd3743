"""Q8_0 stacks with f32 activations over many rows (prefill chunks, the
lm.pas:391-408 forward over a block of embeddings): the products run on the
bf16 matrix cores (quants exact in bf16, activations split exactly into three
bf16 parts), in 16-row tiles up to 64 rows and in 64-row tiles staged through
LDS above. Every layer's output of every row against the oracle's (the
reference's Q8_0 bar, 1e-3 of max |ref|; QwenDiff of tests/test.tts.qwen.ref.pas),
for chunk sizes that take each tile shape, ragged last tiles and the K-sliced
o_proj / down products, with the context growing across chunks."""
import numpy as np
import pytest

import q3h
import q3o
import synth
from models import rel

pytestmark = pytest.mark.gpu


# chunks of one context: 16-row tiles (TM 1, 2, 4) and 64-row tiles staged in
# LDS (65 = one full tile and one row, 130 = two and two rows, 200)
@pytest.mark.parametrize("chunks", [(5, 17, 48), (33, 65, 130), (64, 200, 1)],
                         ids=["tiles16", "tiles64", "big_then_decode"])
def test_q8_prefill_layers_match_the_oracle(device, chunks):
    print(f"case chunks={chunks}", flush=True)
    dims = dict(synth.TALKER, layers=3)
    layers, final = synth.stack_weights(43, "talker.model.", dims, norm_std=0.1,
                                        quantize=q3o.quantize_q8_0)
    st = q3h.Stack(device, dict(dims, dtype=q3h.Q8_0, kv_f16=0, act_q8=0, max_positions=512),
                   layers, final, q3h.Q8_0)
    ost = q3o.Stack(dims, layers, final, q3o.Q8_0, act_q8=0)
    ctx, oc = q3h.Context(st, 512), q3o.Ctx(ost, 512)
    worst = 0.0
    try:
        for i, rows in enumerate(chunks):
            x = synth.prompt(700 + i, rows)
            _, normed, lo, _ = ctx.forward_probe(x)
            onormed, olo = oc.forward(x, layer_out=True)
            for l in range(dims["layers"]):
                r = rel(lo[l], olo[l])
                worst = max(worst, r)
                assert r < 1e-3, (rows, l, r)
            assert rel(normed, onormed) < 1e-3
        assert ctx.length == sum(chunks)
        print(f"worst relative error {worst:.2e}", flush=True)
    finally:
        ctx.destroy()
        oc.destroy()
        st.destroy()
        ost.destroy()


# other shapes: 4 query / 2 kv heads (o_proj K = 512: 2 slices) and an
# intermediate size of 1536 (down: 6 slices); 24 and 40 rows take the
# 256-column slices, 8 rows the whole-K tiles
def test_q8_prefill_other_slice_counts(device):
    dims = dict(synth.TALKER, layers=2, heads=4, kv_heads=2, intermediate=1536)
    layers, final = synth.stack_weights(44, "talker.model.", dims, norm_std=0.1,
                                        quantize=q3o.quantize_q8_0)
    st = q3h.Stack(device, dict(dims, dtype=q3h.Q8_0, kv_f16=0, act_q8=0, max_positions=128),
                   layers, final, q3h.Q8_0)
    ost = q3o.Stack(dims, layers, final, q3o.Q8_0, act_q8=0)
    ctx, oc = q3h.Context(st, 128), q3o.Ctx(ost, 128)
    try:
        for i, rows in enumerate((24, 40, 8)):
            x = synth.prompt(710 + i, rows)
            _, normed, lo, _ = ctx.forward_probe(x)
            onormed, olo = oc.forward(x, layer_out=True)
            for l in range(dims["layers"]):
                assert rel(lo[l], olo[l]) < 1e-3, (rows, l, rel(lo[l], olo[l]))
            assert rel(normed, onormed) < 1e-3
    finally:
        ctx.destroy()
        oc.destroy()
        st.destroy()
        ost.destroy()
