"""q3h_forward_embeds_probe: the raw output of every layer and the final-normed
state of every row, as TQwenLm's probe reports them to the reference's tests
(TOnQwenProbe, lm.pas:139-142, 380-389: name.layerN and name.out; compared
layer by layer in tests/test.tts.qwen.lm.pas:211-249). Here: the f32 stack's
layers and normed rows against the transformers goldens at 1e-4, the Q8_0 and
int8 stacks' against the oracle's (1e-3; bit for bit on the int8 path), and
the probed call's outputs equal to the plain call's."""
import os

import numpy as np
import pytest

import q3h
import q3o
import synth
from models import rel

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.mark.parametrize("name", ["qwen3_small_3l", "qwen3_full_2l"])
def test_probe_layers_match_transformers(device, name):
    print(f"case {name}", flush=True)
    g = np.load(os.path.join(GOLDEN, name + ".npz"))
    L, H, heads, kvh, hd, inter = g["dims"].tolist()
    dims = dict(layers=L, hidden=H, heads=heads, kv_heads=kvh, head_dim=hd, intermediate=inter,
                rms_eps=1e-6, rope_theta=1e6)
    layers, final = synth.stack_weights(int(g["seed"]), "golden.", dims, std=float(g["std"]),
                                        norm_std=float(g["norm_std"]))
    st = q3h.Stack(device, dict(dims, dtype=q3h.F32, kv_f16=0, act_q8=0, max_positions=64),
                   layers, final, q3h.F32)
    ctx = q3h.Context(st, 64)
    try:
        pos = 0
        for rows in g["schedule"].tolist():
            _, normed, lo, nr = ctx.forward_probe(g["x"][pos:pos + rows])
            for l in range(L - 1):  # the goldens keep every layer's output but the last
                want = g["raw"][l][pos:pos + rows]
                assert rel(lo[l], want) < 1e-4, (pos, l, rel(lo[l], want))
            # the final-normed state of every row (the probe's name.out)
            assert rel(nr, g["normed"][pos:pos + rows]) < 1e-4, (pos, rel(nr, g["normed"][pos:pos + rows]))
            assert rel(nr[-1], normed) < 1e-6
            pos += rows
            assert rel(normed, g["normed"][pos - 1]) < 1e-4
    finally:
        ctx.destroy()
        st.destroy()


@pytest.mark.parametrize("act_q8", [0, 1], ids=["q8_0", "int8"])
def test_probe_layers_match_the_oracle(device, act_q8):
    dims = dict(synth.TALKER, layers=3)
    layers, final = synth.stack_weights(41, "talker.model.", dims, norm_std=0.1,
                                        quantize=q3o.quantize_q8_0)
    head = q3o.quantize_q8_0(synth.talker_head(41))
    st = q3h.Stack(device, dict(dims, dtype=q3h.Q8_0, kv_f16=0, act_q8=act_q8,
                                max_positions=128), layers, final, q3h.Q8_0)
    st.add_head(head, q3h.Q8_0)
    ost = q3o.Stack(dims, layers, final, q3o.Q8_0, act_q8=act_q8)
    a, b, oc = q3h.Context(st, 128), q3h.Context(st, 128), q3o.Ctx(ost, 128)
    try:
        for i, rows in enumerate((20, 1, 1)):
            x = synth.prompt(600 + i, rows)
            lg, normed, lo, nr = a.forward_probe(x, head=0)
            lg2, normed2 = b.forward(x, head=0)
            assert np.array_equal(lg, lg2) and np.array_equal(normed, normed2)  # probing changes nothing
            onormed, olo = oc.forward(x, layer_out=True)
            for l in range(dims["layers"]):
                if act_q8:
                    assert np.array_equal(lo[l], olo[l]), (i, l)
                else:
                    assert rel(lo[l], olo[l]) < 1e-3, (i, l, rel(lo[l], olo[l]))
            onr = q3o.rmsnorm_rows(olo[-1], final)
            assert nr.shape == (rows, dims["hidden"])
            if act_q8:
                assert np.array_equal(nr, onr), i
            else:
                assert rel(nr, onr) < 1e-3, (i, rel(nr, onr))
            assert rel(nr[-1], normed) < 1e-6
    finally:
        for c in (a, b, oc):
            c.destroy()
        st.destroy()
        ost.destroy()
