"""Seeded synthetic inputs of the Qwen3-TTS frame step.

Weights and embeddings are N(0, std) float32 from numpy's PCG64 with one
stream per tensor: SeedSequence([seed, crc32(name)]), so any tensor can be
regenerated alone. Norm weights are 1 by default (the benchmark
configurations); tests may ask for 1 + N(0, norm_std) to exercise them.
Model dimensions follow tests/data/infer-ref/qwen3-tts-lm/manifest.json
("stacks") of the reference: hidden 1024, 16 / 8 heads of 128, FFN 3072,
eps 1e-6, RoPE theta 1e6; talker 28 layers and 3072 codes, code predictor 5
layers and 15 heads of 2048 codes.
"""
import zlib

import numpy as np

TALKER = dict(layers=28, hidden=1024, heads=16, kv_heads=8, head_dim=128, intermediate=3072,
              rms_eps=1e-6, rope_theta=1e6)
PREDICTOR = dict(TALKER, layers=5)
VOCAB = 3072
CP_VOCAB = 2048
GROUPS = 16


def normal(seed, name, shape, std=0.02):
    rng = np.random.Generator(np.random.PCG64(np.random.SeedSequence(
        [int(seed) & 0xFFFFFFFF, zlib.crc32(name.encode())])))
    a = rng.standard_normal(size=shape, dtype=np.float32)
    if std != 1.0:
        a *= np.float32(std)
    return a


def norm_vector(seed, name, n, norm_std):
    if norm_std == 0:
        return np.ones(n, dtype=np.float32)
    return (1.0 + normal(seed, name, (n,), norm_std)).astype(np.float32)


def layer_weights(seed, prefix, dims, l, std=0.02, norm_std=0.0):
    """f32 weights of layer l: matrices [out][in] and norm vectors."""
    H, hd = dims["hidden"], dims["head_dim"]
    NQ, NKV, I = dims["heads"] * hd, dims["kv_heads"] * hd, dims["intermediate"]
    p = f"{prefix}layers.{l}."
    return {
        "wq": normal(seed, p + "self_attn.q_proj.weight", (NQ, H), std),
        "wk": normal(seed, p + "self_attn.k_proj.weight", (NKV, H), std),
        "wv": normal(seed, p + "self_attn.v_proj.weight", (NKV, H), std),
        "wo": normal(seed, p + "self_attn.o_proj.weight", (H, NQ), std),
        "wgate": normal(seed, p + "mlp.gate_proj.weight", (I, H), std),
        "wup": normal(seed, p + "mlp.up_proj.weight", (I, H), std),
        "wdown": normal(seed, p + "mlp.down_proj.weight", (H, I), std),
        "input_norm": norm_vector(seed, p + "input_layernorm.weight", H, norm_std),
        "post_norm": norm_vector(seed, p + "post_attention_layernorm.weight", H, norm_std),
        "q_norm": norm_vector(seed, p + "self_attn.q_norm.weight", hd, norm_std),
        "k_norm": norm_vector(seed, p + "self_attn.k_norm.weight", hd, norm_std),
    }


MATRICES = ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown")


def stack_weights(seed, prefix, dims, std=0.02, norm_std=0.0, quantize=None):
    """(layers, final_norm); quantize: None (f32) or a function f32 -> Q8_0
    blocks applied to each matrix as it is generated (keeps the peak memory
    at one f32 matrix)."""
    layers = []
    for l in range(dims["layers"]):
        L = layer_weights(seed, prefix, dims, l, std, norm_std)
        if quantize is not None:
            for k in MATRICES:
                L[k] = quantize(L[k])
        layers.append(L)
    final = norm_vector(seed, prefix + "norm.weight", dims["hidden"], norm_std)
    return layers, final


def talker_head(seed, std=0.02):
    return normal(seed, "talker.codec_head.weight", (VOCAB, TALKER["hidden"]), std)


def cp_head(seed, g, std=0.02):
    return normal(seed, f"talker.code_predictor.lm_head.{g}.weight",
                  (CP_VOCAB, TALKER["hidden"]), std)


def codec_embedding(seed, std=0.02):
    return normal(seed, "talker.model.codec_embedding.weight", (VOCAB, TALKER["hidden"]), std)


def pred_embedding(seed, g, std=0.02):
    return normal(seed, f"talker.code_predictor.model.codec_embedding.{g}.weight",
                  (CP_VOCAB, TALKER["hidden"]), std)


def tts_pad(seed, std=0.02):
    return normal(seed, "tts_pad", (TALKER["hidden"],), std)


TEXT_VOCAB = 151936  # talker text_vocab_size
TEXT_HIDDEN = 2048   # talker text_hidden_size


def to_bf16_bits(x):
    """float32 -> bfloat16 bits (round to nearest even), uint16."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def text_projection(seed, text_vocab=TEXT_VOCAB, std=0.02, emb_std=1.0):
    """The text embedding as BF16 bits [text_vocab][2048] (N(0, emb_std)) and
    the projection fc1 [2048][2048] + b1, fc2 [1024][2048] + b2 in f32
    (talker.model.text_embedding, talker.text_projection.linear_fc1 / fc2)."""
    TH, H = TEXT_HIDDEN, TALKER["hidden"]
    emb = np.empty((text_vocab, TH), dtype=np.uint16)
    step = 8192  # rows per chunk: bounded peak memory for the full table
    for r0 in range(0, text_vocab, step):
        n = min(step, text_vocab - r0)
        emb[r0:r0 + n] = to_bf16_bits(normal(seed, f"talker.model.text_embedding.{r0}",
                                             (n, TH), emb_std))
    w1 = normal(seed, "talker.text_projection.linear_fc1.weight", (TH, TH), std)
    b1 = normal(seed, "talker.text_projection.linear_fc1.bias", (TH,), std)
    w2 = normal(seed, "talker.text_projection.linear_fc2.weight", (H, TH), std)
    b2 = normal(seed, "talker.text_projection.linear_fc2.bias", (H,), std)
    return emb, w1, b1, w2, b2


def prompt(seed, rows, hidden=1024, name="prompt"):
    """fp32 N(0, 1) prompt embeddings."""
    return normal(seed, name, (rows, hidden), 1.0)


def lcg_rows(count, seed=12345):
    """The pseudo-random inputs of tests/test.tts.qwen.vulkan.pas:189-199:
    seed := seed*1664525 + 1013904223 (32-bit), x := ((seed shr 8)/2^24 - 0.5)*0.2."""
    out = np.empty(count, dtype=np.float32)
    s = seed & 0xFFFFFFFF
    for i in range(count):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32((np.float64(s >> 8) / (1 << 24) - 0.5) * 0.2)
    return out, s


CODEC_LATENT = 1024
CODEC_DIM = 1536
CODEC_RATES = (8, 5, 4, 3)
FRAME_SAMPLES = 1920


def codec_weights(seed):
    """The back part of the 12 Hz decoder (decoder.* tensors of the speech
    tokenizer) in their safetensors layouts, f32, scaled so that activations
    stay of order one through the blocks (convolutions N(0, 1 / fan_in) times
    a factor, SnakeBeta log-parameters N(0, 0.1), ConvNeXt gamma 0.1)."""
    L, D = CODEC_LATENT, CODEC_DIM

    def n(name, shape, std):
        return normal(seed, "codec." + name, shape, std)

    w = dict(up_w=[], up_b=[], dw_w=[], dw_b=[], norm_w=[], norm_b=[], pw1_w=[], pw1_b=[],
             pw2_w=[], pw2_b=[], gamma=[])
    for i in range(2):
        p = f"upsample.{i}."
        w["up_w"].append(n(p + "0.conv.weight", (L, L, 2), 1.0 / np.sqrt(L)))
        w["up_b"].append(n(p + "0.conv.bias", (L,), 0.01))
        w["dw_w"].append(n(p + "1.dwconv.conv.weight", (L, 1, 7), 0.5 / np.sqrt(7)))
        w["dw_b"].append(n(p + "1.dwconv.conv.bias", (L,), 0.01))
        w["norm_w"].append((1.0 + n(p + "1.norm.weight", (L,), 0.1)).astype(np.float32))
        w["norm_b"].append(n(p + "1.norm.bias", (L,), 0.1))
        w["pw1_w"].append(n(p + "1.pwconv1.weight", (4 * L, L), 1.0 / np.sqrt(L)))
        w["pw1_b"].append(n(p + "1.pwconv1.bias", (4 * L,), 0.01))
        w["pw2_w"].append(n(p + "1.pwconv2.weight", (L, 4 * L), 1.0 / np.sqrt(4 * L)))
        w["pw2_b"].append(n(p + "1.pwconv2.bias", (L,), 0.01))
        w["gamma"].append((0.1 + n(p + "1.gamma", (L,), 0.02)).astype(np.float32))
    w["conv0_w"] = n("decoder.0.conv.weight", (D, L, 7), 1.0 / np.sqrt(7 * L))
    w["conv0_b"] = n("decoder.0.conv.bias", (D,), 0.01)
    w["block"] = []
    for i, rate in enumerate(CODEC_RATES):
        cin, cout = D >> i, D >> (i + 1)
        p = f"decoder.{i + 1}.block."
        b = dict(act_alpha=n(p + "0.alpha", (cin,), 0.1), act_beta=n(p + "0.beta", (cin,), 0.1),
                 up_w=n(p + "1.conv.weight", (cin, cout, 2 * rate), 1.0 / np.sqrt(2 * cin)),
                 up_b=n(p + "1.conv.bias", (cout,), 0.01), res=[])
        for r in range(3):
            q = f"{p}{r + 2}."
            b["res"].append(dict(
                a1_alpha=n(q + "act1.alpha", (cout,), 0.1), a1_beta=n(q + "act1.beta", (cout,), 0.1),
                c1_w=n(q + "conv1.conv.weight", (cout, cout, 7), 0.5 / np.sqrt(7 * cout)),
                c1_b=n(q + "conv1.conv.bias", (cout,), 0.01),
                a2_alpha=n(q + "act2.alpha", (cout,), 0.1), a2_beta=n(q + "act2.beta", (cout,), 0.1),
                c2_w=n(q + "conv2.conv.weight", (cout, cout, 1), 0.5 / np.sqrt(cout)),
                c2_b=n(q + "conv2.conv.bias", (cout,), 0.01)))
        w["block"].append(b)
    w["out_alpha"] = n("decoder.5.alpha", (D >> 4,), 0.1)
    w["out_beta"] = n("decoder.5.beta", (D >> 4,), 0.1)
    w["out_w"] = n("decoder.6.conv.weight", (1, D >> 4, 7), 0.05 / np.sqrt(7 * (D >> 4)))
    w["out_b"] = n("decoder.6.conv.bias", (1,), 0.01)
    return w
