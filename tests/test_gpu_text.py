"""The text projection and the device-side Start on the GPU, through the C ABI,
against the oracle (TQwenTalker.TextProject, talker.pas:390-421, and Start,
talker.pas:471-593). Products in f32 on the matrix cores: within 1e-4 of the
oracle (the reference's f32 GPU-vs-CPU bar, tests/test.tts.qwen.vulkan.pas:
226-231); the BF16 widening and the SiLU clamp are exact."""
import numpy as np
import pytest

import q3h
import q3o
import synth
from models import Model, rel

pytestmark = pytest.mark.gpu

TV = 4096  # rows of the synthetic text embedding (the gather does not depend on it)


@pytest.fixture(scope="module")
def tables():
    return synth.text_projection(31, TV)


@pytest.fixture(scope="module")
def proj(device, tables):
    p = q3h.TextProj(device, *tables)
    yield p
    p.destroy()


def _oracle(tables, ids):
    return q3o.text_project(*tables, ids)


@pytest.mark.parametrize("n", [1, 3, 16, 17, 40, 100, 520])
def test_text_project_parity(proj, tables, n):
    # 1..16 rows: 16-row tiles; 17..32: 32-row tiles; 40, 100: 64-row tiles of
    # the K-split kernel; 520: fc1 on the 64-row full-K kernel
    rng = np.random.default_rng(n)
    ids = rng.integers(0, TV, n).astype(np.int32)
    ids[n // 2] = ids[0]  # a repeated token
    print(f"text projection: {n} rows", flush=True)
    y = proj.project(ids)
    ref = _oracle(tables, ids)
    assert y.shape == ref.shape
    assert rel(y, ref) < 1e-4, rel(y, ref)
    # rows are independent: a repeated token gives the same row within the bar
    assert rel(y[n // 2], ref[0]) < 1e-4


def test_text_project_f32_table(device, tables):
    emb = (tables[0][:300].astype(np.uint32) << 16).view(np.float32)
    p = q3h.TextProj(device, emb, *tables[1:])
    try:
        ids = np.array([5, 299, 0, 17, 5], np.int32)
        y = p.project(ids)
        # the same values as the BF16 table: the same results
        ref = _oracle(tables, ids)
        assert rel(y, ref) < 1e-4
    finally:
        p.destroy()


def test_text_project_clamp_exact(device):
    """fc1 = 0: the SiLU input is b1; entries below -80 contribute exactly 0,
    -80 itself v / (1 + e^80); fc2 = [I 0] reads them out."""
    TH, H = 1024, 1024
    b1 = np.zeros(TH, np.float32)
    vals = np.array([-100.0, -80.5, -80.0, -79.5, 0.0, 5.0, 1.0, -3.0], np.float32)
    b1[:8] = vals
    w1 = np.zeros((TH, TH), np.float32)
    w2 = np.zeros((H, TH), np.float32)
    w2[np.arange(H), np.arange(H)] = 1.0
    b2 = np.zeros(H, np.float32)
    emb = np.ones((4, TH), np.float32)
    p = q3h.TextProj(device, emb, w1, b1, w2, b2)
    try:
        y = p.project([2, 3])
    finally:
        p.destroy()
    for r in range(2):
        assert y[r, 0] == 0.0 and y[r, 1] == 0.0 and y[r, 4] == 0.0
        v = vals[2:].astype(np.float64)
        exact = v / (1.0 + np.exp(-v))
        got = y[r, 2:8].astype(np.float64)
        nz = exact != 0
        assert np.all(np.abs(got[nz] - exact[nz]) <= 1e-6 * np.abs(exact[nz])), (got, exact)
        assert np.all(y[r, 8:] == 0.0)


def test_text_project_errors(proj):
    assert proj.project(np.zeros(0, np.int32)).shape == (0, 1024)
    for bad in ([TV], [-1], [0, 1, TV + 5]):
        with pytest.raises(q3h.Q3HError) as e:
            proj.project(bad)
        assert e.value.code == q3h.E_ARG and "out of range" in str(e.value)
    # the object still works after the errors
    y = proj.project([7])
    assert np.isfinite(y).all()


CODEC = dict(codec_pad=2148, codec_bos=2149)


def _ids(seed, n_text):
    rng = np.random.default_rng(seed)
    role = [3000, 77, 198]
    text = rng.integers(0, TV, n_text).tolist()
    return role + text + [3001, 198, 3000, 77, 198]


def test_frame_start_text(device, tables):
    """Two streams started from token ids on the device (non-streaming and
    streaming, with a speaker and a language id) against the oracle's Start
    rows fed to the oracle frame: prefill state within 1e-4, then identical
    codes through the trailing rows and past them."""
    tts = dict(tts_bos=4090, tts_eos=4091, tts_pad=4092)
    m = Model(device, seed=41, talker_layers=2, cp_layers=1, dtype=q3h.F32, norm_std=0.1,
              max_positions=128)
    p = q3h.TextProj(device, *tables)
    fr = m.frame(n_streams=2, max_positions=128, max_frames=16)
    ofs = []
    try:
        cases = [(True, _ids(1, 12), [2155, 2156, 2050, 2157, 3001, 2148, 2149]),
                 (False, _ids(2, 5), [2154, 2156, 2157, 2148, 2149])]
        for s, (ns, ids, codec) in enumerate(cases):
            print(f"start_text stream {s}: non_streaming={ns}, {len(ids)} ids", flush=True)
            fr.start_text(s, p, ids, codec, non_streaming=ns, **tts, **CODEC)
            pre, trail = q3o.start_rows(lambda t: _oracle(tables, t), m.codec_emb, ids, codec,
                                        tts["tts_bos"], tts["tts_eos"], tts["tts_pad"],
                                        CODEC["codec_pad"], CODEC["codec_bos"], ns)
            of = m.oracle_frame(max_positions=128)
            of.start(pre, trail)
            ofs.append(of)
            lg, past = fr.state(s)
            olg, opast = of.state()
            assert rel(lg, olg) < 1e-4 and rel(past, opast) < 1e-4, (s, rel(lg, olg))
        for i in range(6):  # stream 1 has 5 trailing rows
            codes, alive = fr.step()
            print(f"frame {i}", flush=True)
            for s, of in enumerate(ofs):
                ref = of.next()
                assert np.array_equal(codes[s], ref), (i, s, codes[s], ref)
                lg, _ = fr.state(s)
                olg, _ = of.state()
                assert rel(lg, olg) < 1e-4, (i, s, rel(lg, olg))
    finally:
        fr.destroy()
        for of in ofs:
            of.destroy()
        p.destroy()
        m.destroy()


def test_frame_start_text_errors(device, tables):
    m = Model(device, seed=42, talker_layers=1, cp_layers=1, dtype=q3h.F32, max_positions=32)
    p = q3h.TextProj(device, *tables)
    fr = m.frame(n_streams=1, max_positions=32, max_frames=4)
    tts = dict(tts_bos=1, tts_eos=2, tts_pad=3)
    codec = [2154, 2156, 2157, 2148, 2149]
    try:
        def code(ids, cdc=codec, ns=True, **kw):
            args = dict(tts, **CODEC)
            args.update(kw)
            with pytest.raises(q3h.Q3HError) as e:
                fr.start_text(0, p, ids, cdc, non_streaming=ns, **args)
            return e.value.code
        assert code([1] * 8) == q3h.E_ARG  # no text
        assert code(_ids(3, 2)[:-1] + [TV]) == q3h.E_ARG  # text id out of range
        assert code(_ids(3, 2), cdc=[2154, 3072]) == q3h.E_ARG  # codec id out of range
        assert code(_ids(3, 2), tts_pad=TV) == q3h.E_ARG
        assert code(_ids(3, 6), ns=False) == q3h.E_ARG  # 6 trailing rows > max_frames 4
        assert code(_ids(3, 24)) == q3h.E_CAPACITY  # 3 + 4 + 25 + 1 rows > 32 positions
        # a good start after the errors
        fr.start_text(0, p, _ids(3, 2), codec, non_streaming=True, **tts, **CODEC)
        codes, alive = fr.step()
        assert alive[0] == 1 and (codes[0] >= 0).all()
    finally:
        fr.destroy()
        p.destroy()
        m.destroy()
