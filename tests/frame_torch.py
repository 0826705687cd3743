"""TQwenTalker.NextFrame (mormot.ai.tts.qwen.talker.pas:640-681) composed in
Python over the third-party transformers Qwen3 decoder (float32, CPU, eager
attention) as the stack: an implementation of the frame step that shares
nothing with the oracle's C code. Used by the tests to pin the oracle's
composition with real (random) weights: the code-predictor input
[fPastHidden; codec_emb[code 0]] at positions 0 and 1 of a context reset for
every frame, pred_emb[g - 1][code g] at position g + 1 with head g, the
16-row sum plus the trailing text row (tts_pad once the trailing rows are
used) as the next talker row, and the talker's K/V carried across frames."""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from make_qwen3_golden import build_model  # noqa: E402
from choosers import choose_code0  # noqa: E402


class TorchStack:
    """One transformers Qwen3Model and its K/V cache: forward(rows) appends
    rows at the next positions and returns the final-normed last row."""

    def __init__(self, dims, layers, final):
        from transformers import DynamicCache
        self._cache_cls = DynamicCache
        self.m = build_model(dims, layers, final)
        self.reset()

    def reset(self):
        self.cache = self._cache_cls(config=self.m.config)
        self.pos = 0

    def forward(self, rows):
        rows = np.asarray(rows, np.float32)
        n = rows.shape[0]
        with torch.no_grad():
            out = self.m(inputs_embeds=torch.from_numpy(rows)[None], past_key_values=self.cache,
                         use_cache=True, position_ids=torch.arange(self.pos, self.pos + n)[None])
        self.pos += n
        return out.last_hidden_state[0, -1].numpy().astype(np.float32)


class TorchFrame:
    """The frame step over two TorchStacks and the f32 tables and heads."""

    def __init__(self, talker, cp, talker_head, cp_heads, codec_emb, pred_emb, tts_pad,
                 eos=-1, penalty=1.05):
        self.t, self.c = talker, cp
        self.th, self.ch = talker_head, cp_heads
        self.codec_emb, self.pred_emb, self.tts_pad = codec_emb, pred_emb, tts_pad
        self.eos, self.penalty = eos, penalty
        self.groups = len(pred_emb) + 1

    def start(self, prefill, trailing):
        self.t.reset()
        self.past = self.t.forward(prefill)
        self.logits = (self.th @ self.past).astype(np.float32)
        self.trailing = trailing
        self.history = []
        self.step = 0

    def next(self):
        code = choose_code0(self.logits, self.eos, self.history, self.penalty)
        if code == self.eos:
            return None
        self.history.append(code)
        codes = [code]
        self.c.reset()
        x = self.c.forward(np.stack([self.past, self.codec_emb[code]]))
        self.cp_logits = []
        for g in range(self.groups - 1):
            if g > 0:
                x = self.c.forward(self.pred_emb[g - 1][codes[g]][None])
            lg = (self.ch[g] @ x).astype(np.float32)
            self.cp_logits.append(lg)
            codes.append(int(np.argmax(lg)))  # the first maximum
        row = self.codec_emb[code].copy()
        for g in range(1, self.groups):
            row = row + self.pred_emb[g - 1][codes[g]]
        if self.step < len(self.trailing):
            row = row + self.trailing[self.step]
        else:
            row = row + self.tts_pad
        self.row = row
        self.past = self.t.forward(row[None])
        self.logits = (self.th @ self.past).astype(np.float32)
        self.step += 1
        return np.array(codes, np.int32)
