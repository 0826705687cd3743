"""q3h_forward_embeds_noalloc (no counterpart in the reference: for callers
that cannot allocate device memory) against q3h_forward_embeds, through the
C ABI: the same rows into two contexts of one stack, one through each entry
point, two calls and more in a row (the second with fewer rows), and the
outputs must be equal bit for bit - the same kernels on the same inputs, only
the work buffers differ (the device's static scratch array instead of the
context's own). Also: the limits are errors, and a failed call leaves the
context as it was."""
import ctypes

import numpy as np
import pytest

import q3h
import q3o
import synth

pytestmark = pytest.mark.gpu

VARIANTS = {
    "q8_f32_act": dict(dtype=q3h.Q8_0, act_q8=0),
    "q8_int8_act": dict(dtype=q3h.Q8_0, act_q8=1),
    "f32": dict(dtype=q3h.F32, act_q8=0),
}


@pytest.mark.parametrize("name", list(VARIANTS))
def test_noalloc_equals_forward(device, name):
    v = VARIANTS[name]
    print(f"noalloc {name}", flush=True)
    dims = dict(synth.TALKER, layers=2)
    q = q3o.quantize_q8_0 if v["dtype"] == q3h.Q8_0 else None
    layers, final = synth.stack_weights(23, "talker.model.", dims, norm_std=0.1, quantize=q)
    head = synth.talker_head(23)
    src = v["dtype"]
    st = q3h.Stack(device, dict(dims, dtype=v["dtype"], kv_f16=0, act_q8=v["act_q8"],
                                max_positions=256), layers, final, src)
    st.add_head(q(head) if q else head, src)
    a, b = q3h.Context(st, 256), q3h.Context(st, 256)
    try:
        # 40 rows, then fewer: 1, 3, 1 (each call's buffers carved again)
        for i, rows in enumerate((40, 1, 3, 1)):
            x = synth.prompt(500 + i, rows)
            la, na = a.forward(x, head=0)
            lb, nb = b.forward(x, head=0, noalloc=True)
            assert np.array_equal(la, lb) and np.array_equal(na, nb), (name, i, rows)
            assert a.length == b.length
        # no head, no outputs
        x = synth.prompt(510, 2)
        a.forward(x, head=-1, want_normed=False)
        b.forward(x, head=-1, want_normed=False, noalloc=True)
        la, na = a.forward(synth.prompt(511, 1), head=0)
        lb, nb = b.forward(synth.prompt(511, 1), head=0, noalloc=True)
        assert np.array_equal(la, lb) and np.array_equal(na, nb)
        # the largest call: Q3H_NOALLOC_MAX_ROWS rows into a fresh context
        c, d = q3h.Context(st, 256), q3h.Context(st, 256)
        x = synth.prompt(512, q3h.NOALLOC_MAX_ROWS)
        lc, nc = c.forward(x, head=0)
        ld, nd = d.forward(x, head=0, noalloc=True)
        assert np.array_equal(lc, ld) and np.array_equal(nc, nd)
        c.destroy()
        d.destroy()
    finally:
        a.destroy()
        b.destroy()
        st.destroy()


def test_noalloc_long_context_equals_forward(device):
    """Past 256 positions: one decode row (the attention splits merged in the
    o_proj product), 3 rows (the splits merged into the attention output) and
    a 16-row chunk (causal prefill attention, no split partials), each equal
    bit for bit to q3h_forward_embeds on a context with the same cache."""
    print("noalloc long context", flush=True)
    dims = dict(synth.TALKER, layers=2)
    layers, final = synth.stack_weights(25, "talker.model.", dims, norm_std=0.1,
                                        quantize=q3o.quantize_q8_0)
    st = q3h.Stack(device, dict(dims, dtype=q3h.Q8_0, kv_f16=0, act_q8=0, max_positions=1024),
                   layers, final, q3h.Q8_0)
    st.add_head(q3o.quantize_q8_0(synth.talker_head(25)), q3h.Q8_0)
    a, b = q3h.Context(st, 1024), q3h.Context(st, 1024)
    try:
        pre = synth.prompt(530, 600)
        a.forward(pre, head=-1, want_normed=False)
        b.forward(pre, head=-1, want_normed=False)
        for i, rows in enumerate((1, 3, 16, 1)):
            x = synth.prompt(540 + i, rows)
            la, na = a.forward(x, head=0)
            lb, nb = b.forward(x, head=0, noalloc=True)
            assert np.array_equal(la, lb) and np.array_equal(na, nb), (i, rows)
            assert a.length == b.length
    finally:
        a.destroy()
        b.destroy()
        st.destroy()


def test_noalloc_scratch_overflow(device):
    """15 rows over 16,384 cached positions need about 21 MB of attention
    partials, more than the scratch array holds: Q3H_E_CAPACITY, the context
    unchanged, and the next call that fits still works."""
    print("noalloc overflow", flush=True)
    dims = dict(synth.TALKER, layers=1)
    layers, final = synth.stack_weights(26, "talker.model.", dims)
    L = 16384
    st = q3h.Stack(device, dict(dims, dtype=q3h.Q8_0, kv_f16=0, act_q8=0, max_positions=L + 64),
                   layers, final, q3h.F32)
    c = q3h.Context(st, L + 64)
    try:
        rng = np.random.Generator(np.random.PCG64(26))
        k = rng.standard_normal((1, dims["kv_heads"], L, dims["head_dim"]), dtype=np.float32)
        v = rng.standard_normal((1, dims["kv_heads"], L, dims["head_dim"]), dtype=np.float32)
        c.fill_kv(k, v)
        del k, v
        assert c.length == L
        with pytest.raises(q3h.Q3HError) as e:
            c.forward(synth.prompt(550, 15), noalloc=True)
        assert e.value.code == q3h.E_CAPACITY and "scratch array" in str(e.value)
        assert c.length == L
        _, n1 = c.forward(synth.prompt(551, 16), noalloc=True)  # prefill attention: fits
        assert c.length == L + 16 and np.isfinite(n1).all()
    finally:
        c.destroy()
        st.destroy()


def test_noalloc_limits(device):
    dims = dict(synth.TALKER, layers=1)
    layers, final = synth.stack_weights(24, "talker.model.", dims)
    st = q3h.Stack(device, dict(dims, dtype=q3h.Q8_0, kv_f16=0, act_q8=0, max_positions=128),
                   layers, final, q3h.F32)
    c = q3h.Context(st, 128)
    try:
        x = synth.prompt(520, q3h.NOALLOC_MAX_ROWS + 1)
        with pytest.raises(q3h.Q3HError) as e:
            c.forward(x, noalloc=True)
        assert e.value.code == q3h.E_CAPACITY and "rows exceed" in str(e.value)
        assert c.length == 0
        with pytest.raises(q3h.Q3HError) as e:
            c.forward(synth.prompt(521, 1), head=3, noalloc=True)
        assert e.value.code == q3h.E_ARG
        _, n1 = c.forward(synth.prompt(522, 2), noalloc=True)
        assert c.length == 2 and np.isfinite(n1).all()
        L = q3h.lib()
        assert L.q3h_forward_embeds_noalloc(None, None, 1, -1, None, None) == q3h.E_ARG
        assert L.q3h_forward_embeds_noalloc(c.h, None, 0, -1, None, None) == 0  # rows <= 0
        assert c.length == 2
    finally:
        c.destroy()
        st.destroy()
