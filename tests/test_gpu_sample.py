"""The device sampler in the frame step (TQwenTalker.ChooseCode0 / ChooseCode
with a sampler, talker.pas:595-638) against the oracle's restatement, whose
draw is pinned to the logits warpers of transformers and whose uniforms are
Philox4x64-10 (tests/test_oracle_sample.py). The library and the oracle share
the draw's evaluation order, so equal logits and equal uniforms give equal
codes: on the int8 path (bit-exact logits) every code must match; on the
f32-activation paths the logits agree to ~1e-6, and the codes of the frames
run here match as well."""
import numpy as np
import pytest

import q3h
from models import Model, rel

pytestmark = pytest.mark.gpu

SAMPLING = [
    dict(do_sample=True, temperature=0.9, top_k=50, top_p=1.0, sub_do_sample=True,
         sub_temperature=0.9, sub_top_k=50, sub_top_p=1.0),   # the qwen_tts defaults
    dict(do_sample=True, temperature=0.7, top_k=20, top_p=0.8, sub_do_sample=True,
         sub_temperature=1.2, sub_top_k=0, sub_top_p=1.0),
]


def _run(m, sampling, seed, n_streams, lens, frames, exact):
    fr = m.frame(n_streams=n_streams, max_positions=96, max_frames=frames + 4)
    fr.set_sampling(seed=seed, **sampling)
    ofs = []
    try:
        for s, L in enumerate(lens):
            pre = np.random.default_rng(700 + s).standard_normal((L, 1024)).astype(np.float32)
            fr.start(s, pre)
            of = m.oracle_frame(max_positions=96)
            of.set_sampling(seed=seed, **sampling)
            of.start(pre)
            ofs.append(of)
        out = []
        for i in range(frames):
            codes, alive = fr.step()
            print(f"frame {i}", flush=True)
            for s, of in enumerate(ofs):
                ref = of.next()
                assert alive[s] == 1
                assert np.array_equal(codes[s], ref), (i, s, codes[s], ref)
                lg, _ = fr.state(s)
                olg, _ = of.state()
                if exact:
                    assert np.array_equal(lg, olg)
                else:
                    assert rel(lg, olg) < 1e-3
            out.append(codes.copy())
        return np.stack(out)
    finally:
        fr.destroy()
        for of in ofs:
            of.destroy()


@pytest.mark.parametrize("k", [0, 1])
def test_sampling_int8_path_bit_exact(device, k):
    m = Model(device, seed=17, talker_layers=2, cp_layers=1, act_q8=1, norm_std=0.1,
              max_positions=96)
    try:
        codes = _run(m, SAMPLING[k], seed=1234 + k, n_streams=4, lens=[20, 33, 17, 40],
                     frames=6, exact=True)
        # all streams share the seed but not the logits: the codes differ
        assert not np.array_equal(codes[:, 0], codes[:, 1])
    finally:
        m.destroy()


@pytest.mark.parametrize("dtype", [q3h.Q8_0, q3h.F32])
def test_sampling_single_stream(device, dtype):
    """One stream: the fused code-predictor path and k_cp_argmax's draw."""
    m = Model(device, seed=19, talker_layers=2, cp_layers=1, dtype=dtype, norm_std=0.1,
              max_positions=96)
    try:
        _run(m, SAMPLING[0], seed=99, n_streams=1, lens=[30], frames=6, exact=False)
    finally:
        m.destroy()


def test_sampling_top_k_1_is_greedy_and_seeds(device):
    m = Model(device, seed=23, talker_layers=2, cp_layers=1, norm_std=0.1, max_positions=96)
    pre = np.random.default_rng(5).standard_normal((24, 1024)).astype(np.float32)
    fr = m.frame(n_streams=2, max_positions=96, max_frames=12)
    try:
        def frames(n=5):
            fr.start(0, pre)
            fr.start(1, pre)
            return np.stack([fr.step()[0].copy() for _ in range(n)])
        greedy = frames()
        fr.set_sampling(True, 0.9, 1, 1.0, True, 0.9, 1, 1.0, seed=0)
        assert np.array_equal(frames(), greedy)  # top-k 1: the argmax
        fr.set_sampling(True, 0.9, 50, 1.0, True, 0.9, 50, 1.0, seed=4321)
        a = frames()
        assert np.array_equal(frames(), a)  # a fixed seed: the same sentence again
        assert np.array_equal(a[:, 0], a[:, 1])  # same seed, same logits: same draws
        assert not np.array_equal(a, greedy)
        fr.set_sampling(True, 0.9, 50, 1.0, True, 0.9, 50, 1.0, seed=0)
        b = frames()
        c = frames()
        # seed 0: a fresh seed per start (every stream and sentence its own)
        assert not np.array_equal(b, c) and not np.array_equal(b[:, 0], b[:, 1])
        fr.set_sampling()  # back to greedy
        assert np.array_equal(frames(), greedy)
    finally:
        fr.destroy()
        m.destroy()


def test_sampling_errors(device):
    m = Model(device, seed=29, talker_layers=1, cp_layers=1, max_positions=32)
    fr = m.frame(n_streams=1, max_positions=32, max_frames=4)
    try:
        for bad in (dict(do_sample=True, temperature=0.0), dict(do_sample=True, top_k=-1),
                    dict(do_sample=True, top_p=0.0), dict(do_sample=True, top_p=1.5),
                    dict(do_sample=True, top_k=0, top_p=0.9),
                    dict(sub_do_sample=True, sub_top_k=65, sub_top_p=0.9)):
            with pytest.raises(q3h.Q3HError) as e:
                fr.set_sampling(**bad)
            assert e.value.code == q3h.E_ARG
        # disabled choosers are not checked
        fr.set_sampling(do_sample=False, temperature=0.0)
    finally:
        fr.destroy()
        m.destroy()
