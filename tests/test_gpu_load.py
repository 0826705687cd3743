"""Weights handed over as BF16 (the safetensors rows as stored) and converted
on the device (widened; quantized to Q8_0 for a Q8_0 stack: the conversion
TQwenLmHeads.MatrixRows / QwenLmStack do on the CPU, lm.pas:244-308). A
stack built from BF16 rows equals, to the bit, the stack built from the same
values widened to f32 on the host, and the Q8_0 one equals the stack built
from the oracle's Q8_0 blocks of those values (the ggml quantizer)."""
import numpy as np
import pytest

import q3h
import q3o
import synth

pytestmark = pytest.mark.gpu

DIMS = dict(synth.TALKER, layers=2)


def _widen(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _forward(dev, cfg, layers, final, src, head, head_src, x):
    s = q3h.Stack(dev, cfg, layers, final, src)
    h = s.add_head(head, head_src)
    c = q3h.Context(s, 64)
    try:
        return c.forward(x, head=h)
    finally:
        c.destroy()
        s.destroy()


@pytest.mark.parametrize("dtype", [q3h.Q8_0, q3h.F32])
def test_bf16_rows_equal_widened_rows(device, dtype):
    tl, tf = synth.stack_weights(5, "talker.model.", DIMS, norm_std=0.1)
    bl = [{k: (synth.to_bf16_bits(v) if k.startswith("w") else v) for k, v in L.items()}
          for L in tl]
    wl = [{k: (_widen(v) if k.startswith("w") else v) for k, v in L.items()} for L in bl]
    head_bits = synth.to_bf16_bits(synth.talker_head(5))
    cfg = dict(DIMS, dtype=dtype, kv_f16=0, act_q8=0, max_positions=64)
    x = synth.prompt(9, 20)
    lb, nb = _forward(device, cfg, bl, tf, q3h.BF16, head_bits, q3h.BF16, x)
    lw, nw = _forward(device, cfg, wl, tf, q3h.F32, _widen(head_bits), q3h.F32, x)
    assert np.array_equal(lb, lw) and np.array_equal(nb, nw)
    if dtype == q3h.Q8_0:
        ql = [{k: (q3o.quantize_q8_0(v) if k.startswith("w") else v) for k, v in L.items()}
              for L in wl]
        lq, nq = _forward(device, cfg, ql, tf, q3h.Q8_0,
                          q3o.quantize_q8_0(_widen(head_bits)), q3h.Q8_0, x)
        assert np.array_equal(lb, lq) and np.array_equal(nb, nq)


def test_bf16_source_errors(device):
    cfg = dict(DIMS, layers=1, dtype=q3h.F32, kv_f16=0, act_q8=0, max_positions=64)
    tl, tf = synth.stack_weights(6, "talker.model.", dict(DIMS, layers=1))
    s = q3h.Stack(device, cfg, tl, tf, q3h.F32)
    try:
        with pytest.raises(q3h.Q3HError) as e:
            s.add_head(np.zeros((64, 1024 // 32 * 34), np.uint8), q3h.Q8_0)  # f32 stack
        assert e.value.code == q3h.E_ARG
        with pytest.raises(q3h.Q3HError):
            s.add_head(np.zeros((64, 1024), np.uint16), 7)  # unknown dtype
    finally:
        s.destroy()
