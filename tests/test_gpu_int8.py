"""GPU parity of the int8 path (stacks created with act_q8 = 1: activations
quantized per 32-block, int8 MFMA products) against the oracle's act_q8 mode,
which restates ggml's quantize_row_q8_0_ref + vec_dot_q8_0_q8_0 (the Q8_0
format of lm.pas:259-267).

Bar: bit-exact logits, states and greedy codes. Quantized activations make
the layer outputs discontinuous in their inputs: moved by 1e-7 relative, the
oracle itself moves its logits by about 1e-2 (test_oracle_stack.py measures
it), so a tolerance cannot separate a correct int8 path from a wrong one. The
int8 path therefore evaluates every fp32 value in the oracle's documented
order (the int32 block dots are exact; RMSNorm and softmax sums are double,
whose order does not reach the fp32 results in practice)."""
import numpy as np
import pytest

from models import Model, rel

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small8(device):
    m = Model(device, seed=11, talker_layers=4, cp_layers=2, act_q8=1, norm_std=0.1,
              max_positions=160)
    yield m
    m.destroy()


def test_int8_prefill_then_decode(small8, q3h, q3o, synth):
    """One context: a 40-row prefill (products over 40 rows) then single-row
    decode steps with the head (products over 1 row)."""
    m = small8
    ctx, octx = q3h.Context(m.ts, 64), q3o.Ctx(m.ot, 64)
    try:
        x = synth.prompt(12, 40)
        worst = 0.0
        for step in range(6):
            print(f"int8 step {step} rows {x.shape[0]}", flush=True)
            lg, st = ctx.forward(x, head=0)
            ost = octx.forward(x)
            olg = m.ot.head(m.th, ost)
            r = max(rel(lg, olg), rel(st, ost))
            worst = max(worst, r)
            assert np.array_equal(lg, olg) and np.array_equal(st, ost), (step, r)
            code = int(np.argmax(olg[:2048]))
            x = m.codec_emb[code][None]
        print(f"int8 forward: worst {worst:.2e}")
    finally:
        ctx.destroy()
        octx.destroy()


@pytest.mark.parametrize("n", [3, 20, 32])
def test_int8_batch_rows(small8, q3h, q3o, synth, n):
    """forward_embeds_batch over n contexts of ragged lengths (products over
    n rows: one, two and four 16-row tiles per workgroup paths)."""
    print(f"case n={n}", flush=True)
    m = small8
    rng = np.random.Generator(np.random.PCG64(n))
    lens = rng.integers(1, 30, size=n)
    ctxs = [q3h.Context(m.ts, 64) for _ in range(n)]
    octxs = [q3o.Ctx(m.ot, 64) for _ in range(n)]
    try:
        for i, L in enumerate(lens):
            p = synth.prompt(100 + i, int(L))
            ctxs[i].forward(p, want_logits=False, want_normed=False)
            octxs[i].forward(p)
        for step in range(2):
            x = synth.prompt(200 + step, n)
            lg, normed = q3h.forward_batch(ctxs, x, heads=[0] * n)
            for i in range(n):
                ost = octxs[i].forward(x[i:i + 1])
                olg = m.ot.head(m.th, ost)
                assert np.array_equal(normed[i], ost), (step, i, rel(normed[i], ost))
                assert np.array_equal(lg[i], olg), (step, i, rel(lg[i], olg))
    finally:
        for c in ctxs + octxs:
            c.destroy()


@pytest.mark.parametrize("n", [32, 48])
def test_int8_frame_streams(small8, synth, n):
    """The batched frame step with 32 streams (one slice): code-predictor
    products over 64 rows (the 2-row prefill of every stream) and 32 rows, the
    talker over 32 ragged contexts; and with 48 streams (two slices of 24,
    each its own graph on its own HIP stream)."""
    m = small8
    rng = np.random.Generator(np.random.PCG64(5))
    lens = rng.integers(16, 40, size=n)
    fr = m.frame(n_streams=n, max_positions=64, max_frames=8)
    ofs = []
    try:
        for s, L in enumerate(lens):
            pre = synth.prompt(300 + s, int(L))
            fr.start(s, pre)
            of = m.oracle_frame(max_positions=64)
            of.start(pre)
            ofs.append(of)
        for i in range(4):
            codes, alive = fr.step()
            print(f"frame {i}", flush=True)
            for s, of in enumerate(ofs):
                ref = of.next()
                assert alive[s] == 1
                assert np.array_equal(codes[s], ref), (i, s, codes[s], ref)
                lg, past = fr.state(s)
                olg, opast = of.state()
                assert np.array_equal(lg, olg) and np.array_equal(past, opast), (
                    i, s, rel(lg, olg))
    finally:
        fr.destroy()
        for of in ofs:
            of.destroy()


def test_int8_full_model_16_frames(device, synth):
    """The full shapes (28-layer talker, 5-layer code predictor) with
    quantized activations: 8 streams, 16 frames of identical greedy codes."""
    m = Model(device, seed=13, act_q8=1, max_positions=64)
    rng = np.random.Generator(np.random.PCG64(13))
    lens = rng.integers(16, 25, size=8)
    fr = m.frame(n_streams=8, max_positions=64, max_frames=20)
    ofs = []
    try:
        for s, L in enumerate(lens):
            pre = synth.prompt(400 + s, int(L))
            fr.start(s, pre)
            of = m.oracle_frame(max_positions=64)
            of.start(pre)
            ofs.append(of)
        worst = 0.0
        for i in range(16):
            codes, alive = fr.step()
            for s, of in enumerate(ofs):
                ref = of.next()
                assert alive[s] == 1
                assert np.array_equal(codes[s], ref), (i, s, codes[s], ref)
                lg, past = fr.state(s)
                olg, opast = of.state()
                r = rel(lg, olg)
                worst = max(worst, r)
                assert np.array_equal(lg, olg) and np.array_equal(past, opast), (i, s, r)
            print(f"frame {i}: worst logits difference so far {worst:.2e}", flush=True)
    finally:
        fr.destroy()
        for of in ofs:
            of.destroy()
        m.destroy()


def test_int8_frame_32_streams_long_prompts(device, synth):
    """The batched serving workload's shapes at reduced depth (talker 4
    layers, code predictor 2, real widths): 32 streams with prompt lengths
    uniform in [16, 256] from the workload's generator, 14 frames, so that
    contexts pass 256 positions (more than one round of the attention's key
    loop). The streams start together
    (q3h_frame_start_batch, their prefills overlapping). Bit-exact against the
    oracle."""
    rng = np.random.Generator(np.random.PCG64(1))
    lens = rng.integers(16, 257, size=32)
    frames = 14
    assert lens.max() + frames > 256
    m = Model(device, seed=17, talker_layers=4, cp_layers=2, act_q8=1, norm_std=0.1,
              max_positions=300)
    fr = m.frame(n_streams=32, max_positions=300, max_frames=16)
    ofs = []
    try:
        pres = [synth.prompt(1000 + s, int(L)) for s, L in enumerate(lens)]
        fr.start_batch(list(range(32)), pres)
        for pre in pres:
            of = m.oracle_frame(max_positions=300)
            of.start(pre)
            ofs.append(of)
        for i in range(frames):
            codes, alive = fr.step()
            print(f"frame {i}: longest context {int(lens.max()) + i + 1}", flush=True)
            for s, of in enumerate(ofs):
                ref = of.next()
                assert alive[s] == 1
                assert np.array_equal(codes[s], ref), (i, s, codes[s], ref)
                lg, past = fr.state(s)
                olg, opast = of.state()
                assert np.array_equal(lg, olg) and np.array_equal(past, opast), (
                    i, s, rel(lg, olg))
    finally:
        fr.destroy()
        for of in ofs:
            of.destroy()
        m.destroy()


@pytest.fixture(scope="module")
def small8h(device):
    """The int8 path with half-float K/V caches (the reference's KvF16,
    lm.pas:120-123, 352, which applies to any stack)."""
    m = Model(device, seed=21, talker_layers=4, cp_layers=2, act_q8=1, kv_f16=1, norm_std=0.1,
              max_positions=300)
    yield m
    m.destroy()


def test_int8_f16_cache_prefill_then_decode(small8h, q3h, q3o, synth):
    """int8 products with an f16 cache: a 40-row prefill, then single-row
    decode steps with the head; logits and states bit-exact against the
    oracle with the same cache precision, and the cache itself equal."""
    m = small8h
    ctx, octx = q3h.Context(m.ts, 64), q3o.Ctx(m.ot, 64)
    try:
        x = synth.prompt(31, 40)
        for step in range(8):
            print(f"int8 f16-cache step {step} rows {x.shape[0]}", flush=True)
            lg, st = ctx.forward(x, head=0)
            ost = octx.forward(x)
            olg = m.ot.head(m.th, ost)
            assert np.array_equal(lg, olg) and np.array_equal(st, ost), (
                step, rel(lg, olg), rel(st, ost))
            x = m.codec_emb[int(np.argmax(olg[:2048]))][None]
        for layer in range(m.tdims["layers"]):
            k, v = ctx.read_kv(layer)
            ok, ov = octx.read_kv(layer)
            assert np.array_equal(k, ok) and np.array_equal(v, ov), layer
            # the values are half floats
            assert np.array_equal(k, k.astype(np.float16).astype(np.float32))
    finally:
        ctx.destroy()
        octx.destroy()


def test_int8_f16_cache_frame_32_streams_past_256(small8h, synth):
    """The batched frame step on int8 stacks with f16 caches: 32 streams with
    prompt lengths uniform in [16, 256] (one raised to 252), 10 frames, so
    that contexts pass 256 positions; codes, logits and states bit-exact
    against the oracle."""
    m = small8h
    rng = np.random.Generator(np.random.PCG64(3))
    lens = rng.integers(16, 257, size=32)
    lens[7] = 252
    frames = 10
    assert lens.max() + frames > 256
    fr = m.frame(n_streams=32, max_positions=300, max_frames=16)
    ofs = []
    try:
        for s, L in enumerate(lens):
            pre = synth.prompt(1100 + s, int(L))
            fr.start(s, pre)
            of = m.oracle_frame(max_positions=300)
            of.start(pre)
            ofs.append(of)
        for i in range(frames):
            codes, alive = fr.step()
            print(f"f16 cache frame {i}: longest context {int(lens.max()) + i + 1}", flush=True)
            for s, of in enumerate(ofs):
                ref = of.next()
                assert alive[s] == 1
                assert np.array_equal(codes[s], ref), (i, s, codes[s], ref)
                lg, past = fr.state(s)
                olg, opast = of.state()
                assert np.array_equal(lg, olg) and np.array_equal(past, opast), (
                    i, s, rel(lg, olg))
    finally:
        fr.destroy()
        for of in ofs:
            of.destroy()
