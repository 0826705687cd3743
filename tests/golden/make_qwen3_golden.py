"""Write tests/golden/qwen3_*.npz: golden vectors of a plain Qwen3 decoder stack
fed with embedding rows, from the third-party transformers package installed
in the build container (models/qwen3/modeling_qwen3.py, eager attention, fp32,
CPU). transformers is not the reference; it restates the same published model
(the reference's fixture manifest.json: "plain Qwen3 decoders (per-head q_norm
/ k_norm, SwiGLU, no bias)", generated with transformers' Qwen3 modules).

The weights are not stored: they are regenerated from their seed by
mormot2-qwen-tts_amd/synth.py (numpy PCG64), with random norm weights
(1 + N(0, 0.1)) so that a wrong norm index shows. Stored: the input rows, the
call schedule (rows per call, a K/V cache carried across calls), the raw
output of each layer but the last, and the final-normed state of every row.

Run (build container, no network): python tests/golden/make_qwen3_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "mormot2-qwen-tts_amd"))
import synth  # noqa: E402

CASES = {
    # the real widths (talker / code predictor), 2 layers
    "qwen3_full_2l": dict(dims=dict(synth.TALKER, layers=2), seed=101, schedule=[40, 1, 2],
                          norm_std=0.1, std=0.02),
    # narrow, 3 layers, 4 q heads per kv head
    "qwen3_small_3l": dict(dims=dict(layers=3, hidden=256, heads=8, kv_heads=2, head_dim=128,
                                     intermediate=512, rms_eps=1e-6, rope_theta=1e6),
                           seed=202, schedule=[5, 2, 1], norm_std=0.1, std=0.05),
}


def build_model(dims, layers, final):
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3Model
    cfg = Qwen3Config(vocab_size=16, hidden_size=dims["hidden"],
                      intermediate_size=dims["intermediate"],
                      num_hidden_layers=dims["layers"], num_attention_heads=dims["heads"],
                      num_key_value_heads=dims["kv_heads"], head_dim=dims["head_dim"],
                      rms_norm_eps=dims["rms_eps"], max_position_embeddings=4096,
                      rope_parameters={"rope_type": "default", "rope_theta": dims["rope_theta"]},
                      attention_bias=False, tie_word_embeddings=False)
    cfg._attn_implementation = "eager"
    m = Qwen3Model(cfg).eval()
    with torch.no_grad():
        for l, L in enumerate(layers):
            lay = m.layers[l]
            lay.self_attn.q_proj.weight.copy_(torch.from_numpy(L["wq"]))
            lay.self_attn.k_proj.weight.copy_(torch.from_numpy(L["wk"]))
            lay.self_attn.v_proj.weight.copy_(torch.from_numpy(L["wv"]))
            lay.self_attn.o_proj.weight.copy_(torch.from_numpy(L["wo"]))
            lay.mlp.gate_proj.weight.copy_(torch.from_numpy(L["wgate"]))
            lay.mlp.up_proj.weight.copy_(torch.from_numpy(L["wup"]))
            lay.mlp.down_proj.weight.copy_(torch.from_numpy(L["wdown"]))
            lay.input_layernorm.weight.copy_(torch.from_numpy(L["input_norm"]))
            lay.post_attention_layernorm.weight.copy_(torch.from_numpy(L["post_norm"]))
            lay.self_attn.q_norm.weight.copy_(torch.from_numpy(L["q_norm"]))
            lay.self_attn.k_norm.weight.copy_(torch.from_numpy(L["k_norm"]))
        m.norm.weight.copy_(torch.from_numpy(final))
    return m


def run_case(name, case):
    from transformers import DynamicCache
    dims = case["dims"]
    layers, final = synth.stack_weights(case["seed"], "golden.", dims, std=case["std"],
                                        norm_std=case["norm_std"])
    m = build_model(dims, layers, final)
    total = sum(case["schedule"])
    x = synth.prompt(case["seed"], total, dims["hidden"], name="golden.input")
    cache = DynamicCache(config=m.config)
    normed, raw = [], []
    pos = 0
    with torch.no_grad():
        for rows in case["schedule"]:
            inp = torch.from_numpy(x[pos:pos + rows])[None]
            out = m(inputs_embeds=inp, past_key_values=cache, use_cache=True,
                    output_hidden_states=True,
                    position_ids=torch.arange(pos, pos + rows)[None])
            hs = out.hidden_states
            normed.append(hs[-1][0].numpy())
            raw.append(np.stack([h[0].numpy() for h in hs[1:-1]], 0))
            pos += rows
    np.savez(os.path.join(HERE, name + ".npz"),
             x=x, schedule=np.array(case["schedule"], dtype=np.int32),
             seed=np.array(case["seed"]), std=np.array(case["std"], dtype=np.float32),
             norm_std=np.array(case["norm_std"], dtype=np.float32),
             dims=np.array([dims[k] for k in ("layers", "hidden", "heads", "kv_heads",
                                              "head_dim", "intermediate")], dtype=np.int32),
             normed=np.concatenate(normed, 0),
             raw=np.concatenate(raw, 1))
    print(name, "rows", total, "layers", dims["layers"])


if __name__ == "__main__":
    torch.manual_seed(0)
    for n, c in CASES.items():
        run_case(n, c)
