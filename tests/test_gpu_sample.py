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


def _exact_bucket_head(head):
    """Q8_0 head bytes whose logits put the top 50 in one radix bucket, for
    any hidden state: rows 0-49 all equal to row 200, rows 50-99 its negation,
    every other row's quants 0. One of the two groups has 50 equal positive
    logits, every other logit is 0 or negative, so the first pass of the top-k
    select (sign and exponent) finds a bucket holding exactly the 50 values
    still wanted."""
    b = np.array(head, copy=True)
    blk = b.reshape(b.shape[0], -1, 34)
    src = blk[200].copy()
    neg = src.copy()
    q = neg[:, 2:].view(np.int8)
    q[:] = -q  # the quants lie in [-127, 127]
    blk[0:50] = src
    blk[50:100] = neg
    blk[100:, :, 2:] = 0
    return b


@pytest.mark.parametrize("n_streams", [1, 3])
def test_sampling_top_k_bucket_exact_in_the_first_pass(device, n_streams):
    """The device top-k stops its radix select at the first pass whose bucket
    holds exactly the values still wanted (q3h_sample.h); the oracle takes
    the exact k-th key by sorting. Code-predictor heads 0 and 1 built so that
    the first pass is exact: the codes equal the oracle's and come from the
    positive group."""

    def heads(th, ch):
        ch = list(ch)
        ch[0] = _exact_bucket_head(ch[0])
        ch[1] = _exact_bucket_head(ch[1])
        return th, ch

    m = Model(device, seed=37, talker_layers=2, cp_layers=1, norm_std=0.1, max_positions=96,
              heads=heads)
    try:
        sp = dict(do_sample=True, temperature=0.9, top_k=50, top_p=1.0, sub_do_sample=True,
                  sub_temperature=0.9, sub_top_k=50, sub_top_p=1.0)
        codes = _run(m, sp, seed=4242, n_streams=n_streams, lens=[20, 28, 36][:n_streams],
                     frames=6, exact=False)
        assert np.all((codes[:, :, 1] < 100) & (codes[:, :, 2] < 100)), codes[:, :, 1:3]
        # within the group the draw picks any of the 50 equal logits
        assert len(np.unique(codes[:, :, 1])) > 1
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
