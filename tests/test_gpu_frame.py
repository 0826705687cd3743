"""GPU parity of the frame step (q3h_frame_*) against the oracle's restatement
of TQwenTalker.NextFrame (talker.pas:640-681): identical greedy codes for
every frame, talker logits within 1e-3 (max-abs relative)."""
import numpy as np
import pytest

import q3h
from models import Model, rel

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def full(device):
    m = Model(device, seed=2, max_positions=512)
    yield m
    m.destroy()


def test_frame_b1_q8_16_frames(full, synth):
    """The full frame (28-layer talker, 5-layer code predictor, Q8_0), 48
    prompt rows, 16 frames."""
    m = full
    fr = m.frame(n_streams=1, max_positions=512)
    of = m.oracle_frame(max_positions=512)
    pre = synth.prompt(8, 48)
    trailing = synth.normal(8, "trailing", (3, 1024), 0.02)
    fr.start(0, pre, trailing)
    of.start(pre, trailing)
    lg, past = fr.state(0)
    olg, opast = of.state()
    assert rel(lg, olg) < 1e-3 and rel(past, opast) < 1e-3
    worst = 0.0
    for i in range(16):
        codes, alive = fr.step()
        ref = of.next()
        lg, _ = fr.state(0)
        olg, _ = of.state()
        worst = max(worst, rel(lg, olg))
        print(f"frame {i}: {codes[0].tolist()} rel {rel(lg, olg):.2e}", flush=True)
        assert alive[0] == 1
        assert np.array_equal(codes[0], ref), (i, codes[0], ref)
        assert rel(lg, olg) < 1e-3
    print(f"worst logits error {worst:.2e}")
    fr.destroy()
    of.destroy()


def test_frame_b1_cp_ties_take_the_first_index(device, synth, monkeypatch):
    """Every code-predictor head with rows 2k and 2k + 1 equal, so each logit
    ties with its neighbour: ChooseCode must take the even index of the
    maximal pair. At batch 1 the argmax of heads 0-13 runs inside the next
    q/k/v product, one per wave, and head 14 in its own kernel."""
    orig = synth.cp_head

    def paired(seed, g):
        h = np.array(orig(seed, g), copy=True)
        h[1::2] = h[0::2]
        return h

    monkeypatch.setattr(synth, "cp_head", paired)
    m = Model(device, seed=23, talker_layers=2, cp_layers=2, max_positions=128)
    fr = m.frame(n_streams=1, max_positions=128)
    of = m.oracle_frame(max_positions=128)
    try:
        pre = synth.prompt(23, 20)
        fr.start(0, pre)
        of.start(pre)
        for i in range(4):
            codes, alive = fr.step()
            ref = of.next()
            print(f"frame {i}: {codes[0].tolist()}", flush=True)
            assert alive[0] == 1
            assert np.array_equal(codes[0], ref), (i, codes[0], ref)
            assert np.all(codes[0][1:] % 2 == 0), codes[0]
    finally:
        fr.destroy()
        of.destroy()
        m.destroy()


def test_frame_b1_half_float_kv(device, synth):
    """Half-float K/V caches (the reference's KvF16) on the batch-1 frame:
    the fused code-predictor kernels on f16 caches (the two-row first step and
    the single-row steps) and the talker's f16 attention, against the oracle
    with the same cache rounding."""
    m = Model(device, seed=29, talker_layers=2, cp_layers=2, kv_f16=1, max_positions=128)
    fr = m.frame(n_streams=1, max_positions=128)
    of = m.oracle_frame(max_positions=128)
    try:
        pre = synth.prompt(29, 24)
        fr.start(0, pre)
        of.start(pre)
        for i in range(6):
            codes, alive = fr.step()
            ref = of.next()
            lg, _ = fr.state(0)
            olg, _ = of.state()
            print(f"frame {i}: rel {rel(lg, olg):.2e}", flush=True)
            assert alive[0] == 1
            assert np.array_equal(codes[0], ref), (i, codes[0], ref)
            assert rel(lg, olg) < 1e-3
    finally:
        fr.destroy()
        of.destroy()
        m.destroy()


def test_frame_graph_equals_eager(full, synth):
    m = full
    pre = synth.prompt(9, 20)
    a = m.frame(use_graph=True, max_positions=64)
    b = m.frame(use_graph=False, max_positions=64)
    a.start(0, pre)
    b.start(0, pre)
    for i in range(4):
        ca, _ = a.step()
        cb, _ = b.step()
        assert np.array_equal(ca, cb)
        assert np.array_equal(a.state(0)[0], b.state(0)[0])
    a.destroy()
    b.destroy()


def test_frame_graph_equals_eager_split_attention(full, synth):
    """Past 256 positions the talker's attention runs as splits whose count
    follows the captured cover: a frame launched directly must take the same
    cover, so graph replay and direct launches give the same bits."""
    m = full
    pre = synth.prompt(19, 300)
    a = m.frame(use_graph=True, max_positions=512)
    b = m.frame(use_graph=False, max_positions=512)
    a.start(0, pre)
    b.start(0, pre)
    for i in range(4):
        ca, _ = a.step()
        cb, _ = b.step()
        assert np.array_equal(ca, cb), i
        la, pa = a.state(0)
        lb, pb = b.state(0)
        assert np.array_equal(la, lb), i
        assert np.array_equal(pa, pb), i
    a.destroy()
    b.destroy()


@pytest.fixture(scope="module")
def small(device):
    m = Model(device, seed=3, talker_layers=4, cp_layers=2, norm_std=0.1, max_positions=128)
    yield m
    m.destroy()


def test_frame_start_batch_equals_starts(small, synth, q3h):
    """q3h_frame_start_batch (the prefills of several streams overlapping on
    the device, in any stream order) leaves the states of one q3h_frame_start
    per stream, and the frames that follow give the same codes; a repeated
    stream is refused before anything starts."""
    m = small
    lens = [16, 40, 23, 57]
    pres = [synth.prompt(70 + s, n) for s, n in enumerate(lens)]
    trs = [None, synth.normal(71, "trailing", (2, 1024), 0.02), None,
           synth.normal(73, "trailing", (1, 1024), 0.02)]
    a = m.frame(n_streams=4, max_positions=128)
    b = m.frame(n_streams=4, max_positions=128)
    try:
        for s in range(4):
            a.start(s, pres[s], trs[s])
        order = [3, 1, 0, 2]
        b.start_batch(order, [pres[s] for s in order], [trs[s] for s in order])
        for s in range(4):
            la, pa = a.state(s)
            lb, pb = b.state(s)
            assert np.array_equal(la, lb) and np.array_equal(pa, pb), s
        for i in range(3):
            ca, _ = a.step()
            cb, _ = b.step()
            assert np.array_equal(ca, cb), i
        c = m.frame(n_streams=4, max_positions=128)
        with pytest.raises(q3h.Q3HError) as e:
            c.start_batch([0, 0], [pres[0], pres[1]])
        assert e.value.code == q3h.E_ARG and "repeated" in str(e.value)
        with pytest.raises(q3h.Q3HError) as e:
            c.step()
        assert e.value.code == q3h.E_STATE
        c.destroy()
    finally:
        a.destroy()
        b.destroy()


def test_frame_multi_stream(small, synth):
    m = small
    lens = [16, 40, 23]
    fr = m.frame(n_streams=len(lens), max_positions=128)
    ofs = []
    for s, n in enumerate(lens):
        pre = synth.prompt(60 + s, n)
        tr = synth.normal(60 + s, "trailing", (s + 1, 1024), 0.02)
        fr.start(s, pre, tr)
        of = m.oracle_frame(max_positions=128)
        of.start(pre, tr)
        ofs.append(of)
    for i in range(6):
        codes, alive = fr.step()
        for s, of in enumerate(ofs):
            ref = of.next()
            assert alive[s] == 1
            assert np.array_equal(codes[s], ref), (i, s)
            assert rel(fr.state(s)[0], of.state()[0]) < 1e-3
    fr.destroy()
    for of in ofs:
        of.destroy()


def test_frame_eos_ends_a_stream(small, synth):
    """eos is taken as the code 0 that frame 2 would choose: from then on the
    stream ends, as NextFrame returns false (talker.pas:646-647); eos is
    forbidden before 2 frames (talker.pas:610-611)."""
    m = small
    pre = synth.prompt(70, 12)
    of = m.oracle_frame(max_positions=128)
    of.start(pre)
    first = [of.next()[0] for _ in range(3)]
    of.destroy()
    eos = int(first[2])
    fr = m.frame(n_streams=2, eos=eos, max_positions=128)
    of = m.oracle_frame(eos=eos, max_positions=128)
    fr.start(0, pre)
    fr.start(1, synth.prompt(71, 9))
    of.start(pre)
    ended = None
    for i in range(5):
        codes, alive = fr.step()
        ref = of.next()
        if ref is None:
            ended = i
            assert alive[0] == 0 and np.all(codes[0] == -1)
            break
        assert alive[0] == 1 and np.array_equal(codes[0], ref)
    assert ended is not None and ended >= 2
    # the other stream keeps running
    assert alive[1] == 1
    codes, alive = fr.step()
    assert alive[0] == 0 and alive[1] == 1
    fr.destroy()
    of.destroy()


def test_f32_prefill_512_and_batch8_frames(device, synth):
    """The f32-weight path at the shapes of the batch-8 f32 workload (2 talker
    layers and 1 code-predictor layer at full width): prefills of 512 and
    ragged rows (matrix-core products over 16-row tiles, row counts that are
    not multiples of 16), then batched frames of 8 streams (products over 8
    and 16 rows), against the f32 oracle: identical codes, talker logits and
    states within 1e-4 (the reference's f32 GPU-vs-CPU bar,
    tests/test.tts.qwen.vulkan.pas:226-231)."""
    m = Model(device, seed=21, talker_layers=2, cp_layers=1, dtype=q3h.F32, norm_std=0.1,
              max_positions=600)
    lens = [512, 300, 17, 64, 100, 5, 250, 33]
    fr = m.frame(n_streams=len(lens), max_positions=600, max_frames=8)
    ofs = []
    try:
        for s, n in enumerate(lens):
            print(f"prefill stream {s}: {n} rows", flush=True)
            pre = synth.prompt(500 + s, n)
            fr.start(s, pre)
            of = m.oracle_frame(max_positions=600)
            of.start(pre)
            ofs.append(of)
            lg, past = fr.state(s)
            olg, opast = of.state()
            assert rel(lg, olg) < 1e-4 and rel(past, opast) < 1e-4, (s, rel(lg, olg))
        for i in range(3):
            codes, alive = fr.step()
            print(f"frame {i}", flush=True)
            for s, of in enumerate(ofs):
                ref = of.next()
                assert np.array_equal(codes[s], ref), (i, s, codes[s], ref)
                lg, past = fr.state(s)
                olg, opast = of.state()
                assert rel(lg, olg) < 1e-4 and rel(past, opast) < 1e-4, (i, s, rel(lg, olg))
    finally:
        fr.destroy()
        for of in ofs:
            of.destroy()
        m.destroy()


def _nan_rows(head, rows):
    """Q8_0 head bytes (ggml blocks: fp16 scale, then 32 quants) with every
    block scale of `rows` set to an fp16 NaN: those rows' logits are NaN."""
    b = np.array(head, copy=True)
    blk = b.reshape(b.shape[0], -1, 34)
    blk[rows, :, 0] = 0x00
    blk[rows, :, 1] = 0x7E
    return b


@pytest.mark.parametrize("n_streams", [1, 2])
@pytest.mark.parametrize("sampled", [False, True], ids=["greedy", "sampled"])
def test_frame_nan_logits_keep_codes_in_the_tables(device, synth, n_streams, sampled):
    """NaN logits choose codes by the reference's first-max rule
    (tests/test.tts.qwen.lm.pas:109-117: result 0, moved only on p[i] >
    p[result]), never an index outside the tables. Talker head: logit 0 NaN,
    so code 0 stays. Code-predictor heads: head 0 with logit 5 NaN (a NaN never
    wins), head 1 with logit 0 NaN (code 0), heads 2 and 14 all NaN (code 0;
    head 14's argmax runs in its own kernel at batch 1, heads 0-13 inside the
    next product). Sampled: a NaN key orders above every finite one, so top-k
    keeps it and the weights' sum is NaN: no comparison with the target holds,
    and the walk takes the last positive weight; with every weight NaN (heads 2
    and 14) nothing is drawn and the greedy choice, 0, is the code. Codes equal
    the oracle's, frame for frame."""
    print(f"case n_streams={n_streams} sampled={sampled}", flush=True)

    def heads(th, ch):
        ch = list(ch)
        ch[0] = _nan_rows(ch[0], [5])
        ch[1] = _nan_rows(ch[1], [0])
        ch[2] = _nan_rows(ch[2], slice(None))
        ch[14] = _nan_rows(ch[14], slice(None))
        return _nan_rows(th, [0]), ch

    m = Model(device, seed=31, talker_layers=2, cp_layers=2, max_positions=128, heads=heads)
    fr = m.frame(n_streams=n_streams, max_positions=128)
    sp = dict(do_sample=True, temperature=0.9, top_k=50, top_p=1.0, sub_do_sample=True,
              sub_temperature=0.9, sub_top_k=50, sub_top_p=1.0) if sampled else {}
    fr.set_sampling(seed=77, **sp)
    ofs = []
    try:
        for s in range(n_streams):
            pre = synth.prompt(31 + s, 12 + 5 * s)
            fr.start(s, pre)
            of = m.oracle_frame(max_positions=128)
            of.set_sampling(seed=77, **sp)
            of.start(pre)
            ofs.append(of)
        for i in range(5):
            codes, alive = fr.step()
            print(f"frame {i}: {codes[:, :4].tolist()}", flush=True)
            for s, of in enumerate(ofs):
                ref = of.next()
                assert alive[s] == 1
                assert np.all((codes[s] >= 0) & (codes[s] < 2048)), codes[s]
                assert np.array_equal(codes[s], ref), (i, s, codes[s], ref)
                assert codes[s][3] == 0 and codes[s][15] == 0
                if not sampled:
                    assert codes[s][0] == 0 and codes[s][2] == 0
                lg, _ = fr.state(s)
                olg, _ = of.state()
                assert np.isnan(lg[0]) and np.isnan(olg[0])
                assert rel(lg[1:], olg[1:]) < 1e-3
    finally:
        fr.destroy()
        for of in ofs:
            of.destroy()
        m.destroy()
