"""Pins the oracle's number formats and code choice (CPU only).

- fp16: every finite half value round-trips; random floats (normal, subnormal,
  overflow) convert as numpy's float16 (IEEE round to nearest even).
- Q8_0 (ggml quantize_row_q8_0_ref, named at lm.pas:259-267): closed forms
  (zeros, the amax element is +-127, halfway cases round away from zero), an
  independent numpy restatement on random blocks, the dequantization bound;
  the library's host quantizer gives the same bytes.
- argmax: first max wins (tests/test.tts.qwen.lm.pas:109-117); the reference
  fixture's codes are the argmax of its logits rows (t.lm:131-140).
- ChooseCode0 (talker.pas:595-630): brute-force cases of each processor.
"""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_fp16_all_halves_roundtrip(q3o):
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    f = q3o.fp16_to_fp32(h)
    finite = np.isfinite(f)
    assert np.array_equal(f[finite], h[finite].view(np.float16).astype(np.float32))
    back = q3o.fp32_to_fp16(f[finite])
    # -0 and +0 keep their sign bit
    assert np.array_equal(back, h[finite])


def test_fp16_rounding_matches_numpy(q3o):
    rng = np.random.default_rng(1)
    parts = [rng.standard_normal(200000).astype(np.float32) * s for s in (1e-8, 1e-5, 1.0, 3e4)]
    parts.append(np.array([65504, 65519.99, 65520, 65536, 1e9, 2.0 ** -24, 2.0 ** -25,
                           3 * 2.0 ** -26, 2.0 ** -14 * (1 - 2 ** -12), 0.0, -0.0],
                          dtype=np.float32))
    x = np.concatenate(parts)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(q3o.fp32_to_fp16(x), ref)


def numpy_q8_0(x):
    """Independent restatement of quantize_row_q8_0_ref in numpy float32."""
    b = x.reshape(-1, 32).astype(np.float32)
    amax = np.max(np.abs(b), axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    v = (b * idv[:, None]).astype(np.float32)
    q = (np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))).astype(np.int8)
    out = np.empty((b.shape[0], 34), dtype=np.uint8)
    out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def test_q8_0_zeros(q3o):
    out = q3o.quantize_q8_0(np.zeros((1, 64), np.float32)).reshape(-1)
    assert not out.any()


def test_q8_0_closed_forms(q3o):
    x = np.zeros(32, np.float32)
    x[3] = 127.0  # d = 1, id = 1
    x[4], x[5], x[6], x[7], x[8] = 2.5, -2.5, 0.5, -0.5, 1.49
    x[9] = -127.0
    b = q3o.quantize_q8_0(x[None]).reshape(-1)
    d = b[:2].view(np.float16)[0]
    q = b[2:].view(np.int8)
    assert d == np.float16(1.0)
    assert q[3] == 127 and q[9] == -127
    # halfway cases round away from zero (roundf), not to even
    assert (q[4], q[5], q[6], q[7], q[8]) == (3, -3, 1, -1, 1)


def test_q8_0_amax_is_127(q3o):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((100, 32)).astype(np.float32)
    q = q3o.quantize_q8_0(x).reshape(100, 34)[:, 2:].view(np.int8)
    i = np.argmax(np.abs(x), axis=1)
    assert np.array_equal(np.abs(q[np.arange(100), i]), np.full(100, 127, np.int8))


def test_q8_0_matches_numpy_restatement(q3o):
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(32 * 4000) * s for s in (0.02, 1.0, 1e-6, 300.0)])
    x = x.astype(np.float32)
    got = q3o.quantize_q8_0(x.reshape(-1, 1024)).reshape(-1)
    assert np.array_equal(got, numpy_q8_0(x))


def test_q8_0_dequant_bound(q3o):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((64, 1024)).astype(np.float32) * 0.02
    b = q3o.quantize_q8_0(x)
    y = q3o.dequantize_q8_0(b, 1024)
    blk = b.reshape(-1, 34)
    d16 = blk[:, :2].copy().view(np.float16).astype(np.float64).reshape(-1)
    d = np.max(np.abs(x.reshape(-1, 32)), axis=1).astype(np.float64) / 127
    q = blk[:, 2:].view(np.int8).astype(np.float64)
    bound = d[:, None] / 2 + np.abs(q) * np.abs(d - d16)[:, None] + 1e-12
    assert np.all(np.abs(y.reshape(-1, 32) - x.reshape(-1, 32)) <= bound * (1 + 1e-6))


def test_library_host_quantizer_matches_oracle(q3h, q3o):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((33, 1024)) * 0.02).astype(np.float32)
    x[0] = 0
    x[1, :32] = 2.5
    assert np.array_equal(q3h.quantize_q8_0(x), q3o.quantize_q8_0(x))


def test_argmax_first_max_wins(q3o):
    assert q3o.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert q3o.argmax(np.array([-np.inf, -1, -1], np.float32)) == 1
    assert q3o.argmax(np.array([5], np.float32)) == 0


def test_argmax_nan_rule(q3o):
    """The reference's ArgMax (tests/test.tts.qwen.lm.pas:109-117) keeps
    result 0 and moves only on p[i] > p[result]: a NaN never wins, a NaN p[0]
    keeps 0 (nothing compares greater than it), every value NaN gives 0. The
    device choosers follow the same rule, so a code is always a table row."""
    def ref_argmax(p):  # the Pascal loop, literally
        r = 0
        for i in range(1, len(p)):
            if p[i] > p[r]:
                r = i
        return r
    nan = np.nan
    cases = [[1, nan, 3, 2], [nan, 5, 7], [nan, nan, nan], [-np.inf, nan, -1, -1],
             [2, 2, nan, 2], [nan], [-np.inf, -np.inf]]
    for c in cases:
        p = np.array(c, np.float32)
        assert q3o.argmax(p) == ref_argmax(p), c
    rng = np.random.default_rng(3)
    for _ in range(200):
        p = rng.standard_normal(37).astype(np.float32)
        p[rng.random(37) < 0.2] = np.nan
        assert q3o.argmax(p) == ref_argmax(p)


def test_reference_fixture_codes_are_argmax(q3o):
    f = np.load(os.path.join(GOLDEN, "qwen3_tts_lm_fixture.npz"))
    codes = f["predictor_codes"]
    assert codes.tolist() == [1995, 1642, 988, 1088, 246, 1543, 1579, 437, 1356, 86, 1042, 248,
                              1555, 781, 1772, 374]
    assert q3o.argmax(f["talker_logits_last"][:2048]) == codes[0]
    for g in range(15):
        assert q3o.argmax(f["predictor_logits"][g]) == codes[g + 1]
    # the first code-predictor row is the last normed talker state
    assert np.array_equal(f["predictor_embed"][0], f["talker_norm_last"])


def test_choose_code0_on_reference_fixture(q3o):
    f = np.load(os.path.join(GOLDEN, "qwen3_tts_lm_fixture.npz"))
    lg = f["talker_logits_last"]
    # frame 0: no history, eos forbidden, 2048.. forbidden: code 0 of the fixture
    assert q3o.choose_code0(lg, 2150, [], 1.05) == f["predictor_codes"][0]


def brute_choose_code0(logits, eos, history, penalty):
    v = logits.astype(np.float32).copy()
    V = v.size
    for i in range(V - 1024, V):
        if i != eos:
            v[i] = -np.inf
    if len(history) < 2 and 0 <= eos < V:
        v[eos] = -np.inf
    done = set()
    for i in history:
        if i in done or v[i] == -np.inf:
            continue
        done.add(i)
        s = logits[i]
        v[i] = np.float32(s / np.float32(penalty)) if s > 0 else np.float32(s * np.float32(penalty))
    return int(np.argmax(v))


@pytest.mark.parametrize("case", range(40))
def test_choose_code0_brute_force(q3o, case):
    rng = np.random.default_rng(100 + case)
    V = 1100
    lg = (rng.standard_normal(V) * 0.5).astype(np.float32)
    eos = int(rng.integers(V - 1024, V))
    hist = rng.integers(0, V - 1024, size=int(rng.integers(0, 6))).tolist()
    if case % 3 == 0 and hist:
        hist.append(hist[0])  # a repeated code is penalized once
    if case % 4 == 0:
        lg[eos] = 10.0  # eos wins once allowed
    if case % 5 == 0 and hist:
        lg[hist[0]] = 3.0
        lg[(hist[0] + 1) % (V - 1024)] = 2.9  # the penalty decides
    assert q3o.choose_code0(lg, eos, hist, 1.05) == brute_choose_code0(lg, eos, hist, 1.05)


def test_choose_code0_penalty_once_per_code(q3o):
    V = 1100
    lg = np.zeros(V, np.float32)
    lg[5] = 2.0
    lg[6] = 2.0 / 1.05 ** 2 + 1e-3  # beats 5 only if 5 were penalized twice
    assert q3o.choose_code0(lg, -1, [5, 5], 1.05) == 5
    lg[7] = -1.0
    lg[:] = -2.0
    lg[7] = -1.0
    lg[8] = -1.04
    # a negative logit is multiplied: -1.05 < -1.04
    assert q3o.choose_code0(lg, -1, [7], 1.05) == 8


def test_expf_accuracy_and_special_values(q3o):
    """q3o_expf (Cody-Waite reduction + Taylor series) against double-precision
    exp: < 2 ulp over the range it returns normal numbers, exact at 0, and the
    documented cut-offs (0 below -86, +inf above 88, NaN kept)."""
    x = np.concatenate([np.linspace(-86.0, 88.0, 40001, dtype=np.float32),
                        np.float32([-1e-30, 1e-30, -0.5, 0.5, 0.34657359, -0.34657359])])
    got = q3o.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    err = np.abs(got - ref) / ulp
    assert err.max() < 2.0, (float(err.max()), float(x[np.argmax(err)]))
    assert q3o.expf(np.float32([0.0]))[0] == 1.0
    assert np.all(q3o.expf(np.float32([-86.5, -100.0, -np.inf])) == 0.0)
    assert np.all(np.isposinf(q3o.expf(np.float32([88.5, 1000.0, np.inf]))))
    assert np.isnan(q3o.expf(np.float32([np.nan]))[0])
    # monotone where it matters for the softmax (x <= 0)
    neg = q3o.expf(np.linspace(-20.0, 0.0, 20001, dtype=np.float32))
    assert np.all(np.diff(neg) >= 0)
