"""Pins the oracle's sampler (CPU only).

TQwenTalker draws with TInferSampler (talker.pas:455-469, 626-638), which
lives in the absent mormot2-ai submodule: its random stream cannot be
reproduced, so the draw is pinned by what fixes it independently:
- the uniforms: Philox4x64-10 against the published known answer (counter 0,
  key 0) and against numpy's own Philox bit generator on random counters and
  keys;
- the distribution: for fixed logits and a fine grid of uniforms, the share
  of the grid each code receives equals the probability that the logits
  warpers of the third-party transformers 5.15.0 (TemperatureLogitsWarper,
  TopKLogitsWarper, TopPLogitsWarper, then softmax, in float64) give it;
- closed forms: top-k 1 is the argmax for every uniform (ties at the k-th
  value all kept, as TopKLogitsWarper keeps them); u = 0
  draws the smallest kept index; forbidden (-inf) codes are never drawn;
- the frame: sampling with top-k 1 reproduces the greedy frames.
"""
import numpy as np
import pytest
import torch
from transformers.generation.logits_process import (TemperatureLogitsWarper,
                                                    TopKLogitsWarper, TopPLogitsWarper)


def test_philox_known_answer_and_numpy(q3o):
    # Random123 known-answer vector: philox4x64-10, counter 0, key 0
    assert q3o.philox4x64([0, 0, 0, 0], [0, 0]) == [
        0x16554d9eca36314c, 0xdb20fe9d672d0fdc, 0xd7e772cee186176b, 0x7e68b68aec7ba23b]
    rng = np.random.default_rng(9)
    for _ in range(20):
        ctr = [int(x) for x in rng.integers(0, 1 << 62, 4, dtype=np.uint64)]
        key = [int(x) for x in rng.integers(0, 1 << 63, 2, dtype=np.uint64)]
        key[1] |= 1 << 63  # exercise the top bit
        bg = np.random.Philox(counter=[0, 0, 0, 0], key=[0, 0])
        st = bg.state
        # numpy increments the counter before its first block
        st["state"]["counter"] = np.array([ctr[0] - 1] + ctr[1:], dtype=np.uint64)
        st["state"]["key"] = np.array(key, dtype=np.uint64)
        st["buffer_pos"] = 4
        bg.state = st
        assert [int(x) for x in bg.random_raw(4)] == q3o.philox4x64(ctr, key)


def test_uniforms_are_uniform(q3o):
    u = np.array([q3o.draw_uniform(12345, f, g) for f in range(200) for g in range(16)])
    assert u.min() >= 0.0 and u.max() < 1.0
    # Kolmogorov-Smirnov distance of 3200 draws (p ~ 0.999 bound 1.95 / sqrt(n))
    s = np.sort(u)
    n = len(s)
    ks = max(np.max(np.arange(1, n + 1) / n - s), np.max(s - np.arange(n) / n))
    assert ks < 1.95 / np.sqrt(n)
    # the grid 2^-24: (x >> 40) * 2^-24
    assert np.all(u * (1 << 24) == np.floor(u * (1 << 24)))


def _hf_probs(x, temperature, top_k, top_p):
    s = torch.from_numpy(np.asarray(x, np.float64))[None]
    ids = torch.zeros((1, 1), dtype=torch.long)
    if temperature != 1.0:
        s = TemperatureLogitsWarper(temperature)(ids, s)
    if top_k > 0:
        s = TopKLogitsWarper(top_k)(ids, s)
    if top_p < 1.0:
        s = TopPLogitsWarper(top_p)(ids, s)
    return torch.softmax(s, dim=-1)[0].numpy()


@pytest.mark.parametrize("n,temperature,top_k,top_p", [
    (2048, 1.0, 0, 1.0), (2048, 0.9, 50, 1.0), (3072, 0.9, 50, 1.0), (3072, 0.7, 20, 0.8),
    (2048, 1.3, 64, 0.5), (300, 1.0, 0, 1.0), (1500, 0.5, 10, 1.0)])
def test_sample_distribution_matches_transformers(q3o, n, temperature, top_k, top_p):
    rng = np.random.default_rng(n + top_k)
    x = (rng.standard_normal(n) * 2.0).astype(np.float32)
    if n == 3072:
        x[2048:] = -np.inf  # the talker's forbidden tail
        x[2150] = 1.5       # one allowed code there (eos)
    N = 20000
    grid = (np.arange(N) + 0.5) / N
    counts = np.bincount([q3o.sample(x, temperature, top_k, top_p, float(u)) for u in grid],
                         minlength=n)
    p = _hf_probs(x, temperature, top_k, top_p)
    # a deterministic grid: each code gets its probability to within the grid
    # step (plus the fp32 rounding of the sums)
    assert np.max(np.abs(counts / N - p)) <= 2.0 / N + 1e-5
    assert counts[~np.isfinite(x)].sum() == 0


def test_sample_closed_forms(q3o):
    rng = np.random.default_rng(4)
    x = rng.standard_normal(2048).astype(np.float32)
    x[100] = x.max() + 1.0
    for u in (0.0, 0.3, 0.999999):  # top-k 1: the argmax whatever the uniform
        assert q3o.sample(x, 0.9, 1, 1.0, u) == 100
    x[700] = x[100]  # a tie at the k-th value: both kept (TopKLogitsWarper), half each
    assert [q3o.sample(x, 0.9, 1, 1.0, u) for u in (0.0, 0.49, 0.51, 0.999999)] == [
        100, 100, 700, 700]
    # u = 0: the smallest kept index (top-k 5 keeps these)
    top5 = np.sort(np.argsort(-x, kind="stable")[:5])
    assert q3o.sample(x, 1.0, 5, 1.0, 0.0) == top5[0]
    # top-p so small that only the largest survives
    assert q3o.sample(x, 1.0, 50, 1e-6, 0.77) == 100
    # an all-but-one -inf vector
    y = np.full(3072, -np.inf, np.float32)
    y[1234] = -5.0
    assert all(q3o.sample(y, 0.9, 50, 0.9, u) == 1234 for u in (0.0, 0.5, 0.9999))


def test_sample_without_a_draw_falls_back_to_the_greedy_code(q3o):
    """NaN or +inf scores leave no positive weight (e^(NaN) and e^(inf - inf)
    are NaN): the draw then returns the greedy code of the scores (the
    reference ArgMax rule), never -1, whatever the uniform."""
    x = np.zeros(2048, np.float32)
    x[:] = np.nan
    assert all(q3o.sample(x, 0.9, 50, 1.0, u) == 0 for u in (0.0, 0.5, 0.9999))
    y = np.zeros(3072, np.float32)
    y[77] = np.inf
    assert all(q3o.sample(y, 1.0, 0, 1.0, u) == 77 for u in (0.0, 0.5, 0.9999))
    z = np.linspace(-1, 1, 2048).astype(np.float32)
    z[0] = np.nan
    z[900] = np.inf
    assert q3o.sample(z, 1.0, 0, 1.0, 0.3) == 0  # a NaN first value keeps code 0


def test_frame_sampling_top_k_1_is_greedy(q3o, synth):
    """Sampling with top-k 1 on both choosers reproduces the greedy frames
    (reduced widths so that the oracle runs in a second)."""
    seed = 3
    dims = dict(synth.TALKER, layers=1, hidden=256, heads=4, kv_heads=2, head_dim=64,
                intermediate=512)
    tl, tf = synth.stack_weights(seed, "talker.model.", dims)
    cl, cf = synth.stack_weights(seed, "talker.code_predictor.model.", dims)
    rng = np.random.default_rng(seed)
    th = (rng.standard_normal((3072, 256)) * 0.05).astype(np.float32)
    ch = [(rng.standard_normal((2048, 256)) * 0.05).astype(np.float32) for _ in range(15)]
    ce = (rng.standard_normal((3072, 256)) * 0.02).astype(np.float32)
    pe = [(rng.standard_normal((2048, 256)) * 0.02).astype(np.float32) for _ in range(15)]
    pad = (rng.standard_normal(256) * 0.02).astype(np.float32)
    ot = q3o.Stack(dims, tl, tf, q3o.F32)
    oc = q3o.Stack(dims, cl, cf, q3o.F32)
    pre = rng.standard_normal((6, 256)).astype(np.float32)
    out = []
    for mode in range(3):
        fr = q3o.Frame(ot, oc, th, ch, ce, pe, pad, max_positions=64)
        if mode == 1:
            fr.set_sampling(True, 0.9, 1, 1.0, True, 0.9, 1, 1.0, seed=77)
        elif mode == 2:
            fr.set_sampling(True, 0.9, 50, 1.0, True, 0.9, 50, 1.0, seed=77)
        fr.start(pre)
        out.append(np.array([fr.next() for _ in range(4)]))
        fr.destroy()
    ot.destroy()
    oc.destroy()
    assert np.array_equal(out[0], out[1])
    assert not np.array_equal(out[0], out[2])  # real draws differ from greedy
