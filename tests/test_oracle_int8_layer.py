"""The int8 (act_q8) layer of the oracle, operation by operation, against
numpy: which inputs of the products are quantized, the block products over
them, and what feeds each product.

A Q8_0 stack with Q8_0 activations (ggml quantize_row_q8_0_ref per 32-block,
then vec_dot_q8_0_q8_0: int32 block dots times d_w d_x) runs two calls (3
rows, then 1) through q3o_forward_embeds_traced, which returns every
product's f32 input, the Q8_0 blocks the product read and its output. numpy
then checks, per layer:
  - the blocks of every product input equal numpy's own quantizer of that
    input, byte for byte (q/k/v: the input-normed row; o_proj: the attention
    output; gate / up: the post-attention normed row; down: SwiGLU's output);
  - every product equals the block-integer dot of those bytes with the weight
    blocks, added per 512-column chunk as an fma chain and the chunks in order
    (to the last bit but the double rounding of numpy's fma emulation);
  - every product input follows from the previous outputs by the Qwen3 layer:
    RMSNorm of the residual stream, QK-norm + RoPE + causal GQA softmax over
    the q/k/v outputs (with the K/V of the earlier call), SwiGLU of gate / up;
  - the layer output is h + o + down, each sum rounded once;
and the head reads the quantized final-normed row.
A quantization moved to another point of the layer (before the norm, after
the attention's V, none for o_proj) breaks the byte equality of that product.
"""
import numpy as np
import pytest

import q3o
import synth
from test_oracle_numerics import numpy_q8_0

DIMS = dict(layers=2, hidden=512, heads=4, kv_heads=2, head_dim=128, intermediate=1024,
            rms_eps=1e-6, rope_theta=1e6)


def f32(x):
    return np.asarray(x, np.float32)


def rmsnorm(x, w, eps):
    """ss in double, inv = 1 / sqrt(ss / n + eps) rounded to f32, y = w (x inv)"""
    x = f32(x)
    ss = np.sum(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
    inv = f32(1.0 / np.sqrt(ss / x.shape[-1] + eps))
    return f32(w * f32(x * inv))


def fma32(a, b, c):
    """round_f32(a b + c) through float64 (a b exact here: |a| < 2^20, b f32)"""
    return f32(a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64))


def blocks(b, n):
    """uint8 rows of 34-byte blocks -> (d f32 [.., nb], q int32 [.., nb, 32])"""
    b = np.asarray(b, np.uint8).reshape(b.shape[:-1] + (n // 32, 34))
    d = f32(b[..., :2].copy().view(np.float16)[..., 0])
    q = b[..., 2:].copy().view(np.int8).astype(np.int32)
    return d, q


def int8_product(wb, xb, K):
    """y[m][n]: per 512-column chunk an fma chain acc = fma(dot, d_w d_x,
    acc) over its 16 blocks, the chunk sums added in chunk order"""
    dw, qw = blocks(wb, K)  # [N][nb], [N][nb][32]
    dx, qx = blocks(xb, K)  # [M][nb], [M][nb][32]
    dots = np.einsum("nbk,mbk->mnb", qw, qx)  # exact int32
    sc = f32(dx[:, None, :] * dw[None, :, :])
    nb = K // 32
    acc = np.zeros(dots.shape[:2], np.float32)
    for b0 in range(0, nb, 16):
        part = np.zeros_like(acc)
        for b in range(b0, min(b0 + 16, nb)):
            part = fma32(f32(dots[:, :, b]), sc[:, :, b], part)
        acc = f32(acc + part)
    return acc


def rope(x, pos, theta):
    """rotate_half with the angle pos * inv_freq in f32, cos / sin in double"""
    D = x.shape[-1]
    half = D // 2
    inv = f32(1.0 / np.power(np.float64(theta), np.arange(half, dtype=np.float64) * 2 / D))
    ang = f32(np.float32(pos) * inv)
    c, s = f32(np.cos(ang.astype(np.float64))), f32(np.sin(ang.astype(np.float64)))
    a, b = x[..., :half], x[..., half:]
    return np.concatenate([f32(a * c - b * s), f32(b * c + a * s)], axis=-1)


def attention(q, K, V, scale):
    """causal softmax(q K^T scale) V of one head over K/V [n][D] (double)"""
    sc = (q.astype(np.float64) @ K.astype(np.float64).T) * scale
    w = np.exp(sc - sc.max())
    return w @ V.astype(np.float64) / w.sum()


def close(a, b, tol):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.max(np.abs(a - b)) <= tol * max(np.max(np.abs(b)), 1e-30)


@pytest.fixture(scope="module")
def traced():
    seed = 41
    layers, final = synth.stack_weights(seed, "int8.", DIMS, std=0.05, norm_std=0.1,
                                        quantize=q3o.quantize_q8_0)
    st = q3o.Stack(DIMS, layers, final, q3o.Q8_0, act_q8=1)
    ctx = q3o.Ctx(st, 8)
    x1 = synth.prompt(seed, 3, DIMS["hidden"])
    x2 = synth.prompt(seed + 1, 1, DIMS["hidden"])
    t1 = ctx.forward_traced(x1)
    t2 = ctx.forward_traced(x2)
    head = q3o.quantize_q8_0(synth.normal(seed, "int8.head", (256, DIMS["hidden"]), 0.05))
    logits = st.head(head, t2["normed"])
    yield dict(layers=layers, final=final, calls=[(x1, t1, 0), (x2, t2, 3)], head=head,
               logits=logits)
    ctx.destroy()
    st.destroy()


def test_int8_layer_quantized_inputs_are_exact(traced):
    for x, t, _ in traced["calls"]:
        for l in range(DIMS["layers"]):
            for xn, bn in (("x_qkv", "b_qkv"), ("x_o", "b_o"), ("x_gu", "b_gu"),
                           ("x_down", "b_down")):
                for r in range(x.shape[0]):
                    assert np.array_equal(t[bn][l, r], numpy_q8_0(t[xn][l, r])), (l, r, xn)


def test_int8_layer_products_are_block_integer_dots(traced):
    H, I = DIMS["hidden"], DIMS["intermediate"]
    NQ = DIMS["heads"] * DIMS["head_dim"]
    NKV = DIMS["kv_heads"] * DIMS["head_dim"]
    for x, t, _ in traced["calls"]:
        for l, L in enumerate(traced["layers"]):
            wqkv = np.concatenate([L["wq"], L["wk"], L["wv"]], 0)
            checks = (("y_qkv", wqkv, "b_qkv", H), ("y_o", L["wo"], "b_o", NQ),
                      ("y_gate", L["wgate"], "b_gu", H), ("y_up", L["wup"], "b_gu", H),
                      ("y_down", L["wdown"], "b_down", I))
            for yn, w, bn, K in checks:
                want = int8_product(w, t[bn][l], K)
                got = t[yn][l]
                # float64 fma emulation: equal but for a rare double rounding
                ulp = np.spacing(np.abs(want).max())
                assert np.max(np.abs(got - want)) <= ulp, (l, yn)
                assert np.mean(got == want) > 0.999, (l, yn)
    assert NQ + 2 * NKV == traced["calls"][0][1]["y_qkv"].shape[-1]


def test_int8_layer_inputs_follow_the_qwen3_layer(traced):
    d = DIMS
    H, D, nh, nkv = d["hidden"], d["head_dim"], d["heads"], d["kv_heads"]
    NQ, NKV = nh * D, nkv * D
    eps = d["rms_eps"]
    scale = 1.0 / np.sqrt(D)
    Kc = [[[] for _ in range(nkv)] for _ in range(d["layers"])]
    Vc = [[[] for _ in range(nkv)] for _ in range(d["layers"])]
    for x, t, pos0 in traced["calls"]:
        rows = x.shape[0]
        h = f32(x)
        for l, L in enumerate(traced["layers"]):
            assert close(t["x_qkv"][l], rmsnorm(h, L["input_norm"], eps), 2e-7), l
            y = t["y_qkv"][l]
            att = np.zeros((rows, NQ))
            for r in range(rows):
                pos = pos0 + r
                for g in range(nkv):
                    k = rope(rmsnorm(y[r, NQ + g * D:NQ + (g + 1) * D], L["k_norm"], eps), pos,
                             d["rope_theta"])
                    Kc[l][g].append(k)
                    Vc[l][g].append(y[r, NQ + NKV + g * D:NQ + NKV + (g + 1) * D])
            for r in range(rows):
                n = pos0 + r + 1
                for hh in range(nh):
                    g = hh // (nh // nkv)
                    q = rope(rmsnorm(y[r, hh * D:(hh + 1) * D], L["q_norm"], eps), pos0 + r,
                             d["rope_theta"])
                    att[r, hh * D:(hh + 1) * D] = attention(q, np.array(Kc[l][g][:n]),
                                                            np.array(Vc[l][g][:n]), scale)
            assert close(t["x_o"][l], att, 2e-6), l
            h1 = f32(h + t["y_o"][l])
            assert close(t["x_gu"][l], rmsnorm(h1, L["post_norm"], eps), 2e-7), l
            g_, u = t["y_gate"][l], t["y_up"][l]
            sw = f32(f32(g_ / f32(1.0 + f32(np.exp(-g_.astype(np.float64))))) * u)
            assert close(t["x_down"][l], sw, 1e-6), l
            h = f32(h1 + t["y_down"][l])
            assert np.array_equal(t["layer_out"][l], h), l
        assert close(t["normed"], rmsnorm(h[-1], traced["final"], eps), 2e-7)


def test_int8_head_reads_the_quantized_normed_row(traced):
    t = traced["calls"][-1][1]
    xb = numpy_q8_0(t["normed"])[None]
    want = int8_product(traced["head"], xb, DIMS["hidden"])[0]
    assert np.max(np.abs(traced["logits"] - want)) <= np.spacing(np.abs(want).max())
