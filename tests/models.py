"""Builders shared by the GPU parity tests: the same seeded weights loaded into
the HIP library (through the C ABI) and into the oracle."""
import numpy as np

import q3h
import q3o
import synth


class Model:
    """Talker + code predictor (+ heads, tables) on the device and in the
    oracle, from one seed."""

    def __init__(self, device, seed, talker_layers=28, cp_layers=5, dtype=q3h.Q8_0,
                 act_q8=0, kv_f16=0, norm_std=0.0, max_positions=512, cp_heads=15,
                 heads=None):
        self.seed = seed
        self.dtype = dtype
        self.tdims = dict(synth.TALKER, layers=talker_layers)
        self.cdims = dict(synth.PREDICTOR, layers=cp_layers)
        quant = q3o.quantize_q8_0 if dtype == q3h.Q8_0 else None
        self.tl, self.tf = synth.stack_weights(seed, "talker.model.", self.tdims,
                                               norm_std=norm_std, quantize=quant)
        self.cl, self.cf = synth.stack_weights(seed, "talker.code_predictor.model.", self.cdims,
                                               norm_std=norm_std, quantize=quant)
        q = quant or (lambda a: a)
        self.th = q(synth.talker_head(seed))
        self.ch = [q(synth.cp_head(seed, g)) for g in range(cp_heads)]
        if heads is not None:  # (talker head, code-predictor heads) -> the same, edited
            self.th, self.ch = heads(self.th, self.ch)
        self.codec_emb = synth.codec_embedding(seed)
        self.pred_emb = [synth.pred_embedding(seed, g) for g in range(15)]
        self.tts_pad = synth.tts_pad(seed)
        src = dtype
        tcfg = dict(self.tdims, dtype=dtype, kv_f16=kv_f16, act_q8=act_q8,
                    max_positions=max_positions)
        ccfg = dict(self.cdims, dtype=dtype, kv_f16=kv_f16, act_q8=act_q8, max_positions=16)
        self.ts = q3h.Stack(device, tcfg, self.tl, self.tf, src)
        self.cs = q3h.Stack(device, ccfg, self.cl, self.cf, src)
        self.ts.add_head(self.th, src)
        for h in self.ch:
            self.cs.add_head(h, src)
        odt = q3o.Q8_0 if dtype == q3h.Q8_0 else q3o.F32
        self.ot = q3o.Stack(self.tdims, self.tl, self.tf, odt, kv_f16=kv_f16, act_q8=act_q8)
        self.oc = q3o.Stack(self.cdims, self.cl, self.cf, odt, kv_f16=kv_f16, act_q8=act_q8)

    def oracle_frame(self, eos=-1, max_positions=512):
        return q3o.Frame(self.ot, self.oc, self.th, self.ch, self.codec_emb, self.pred_emb,
                         self.tts_pad, eos=eos, max_positions=max_positions)

    def frame(self, n_streams=1, eos=-1, max_positions=512, use_graph=True, max_frames=64):
        return q3h.Frame(self.ts, self.cs, self.codec_emb, self.pred_emb, self.tts_pad,
                         n_streams=n_streams, eos=eos, max_positions=max_positions,
                         use_graph=use_graph, max_frames=max_frames)

    def destroy(self):
        for o in (self.ts, self.cs, self.ot, self.oc):
            o.destroy()


def rel(a, b):
    """max |a - b| / max |b| (QwenDiff of tests/test.tts.qwen.ref.pas)."""
    return float(np.max(np.abs(np.asarray(a) - np.asarray(b))) / np.max(np.abs(b)))


def top2_margin(logits):
    s = np.sort(np.asarray(logits))
    return float(s[-1] - s[-2])
