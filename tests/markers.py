"""Marker tables: a frame whose composition can be read back exactly.

With every matrix of both stacks zero, a Qwen3 layer adds nothing to its
input (q, k, v, the attention output, o_proj, gate / up and down are all 0),
so a stack returns RMSNorm(its last input row) * final_norm. The frame step of
TQwenTalker.NextFrame (mormot.ai.tts.qwen.talker.pas:640-681) then reduces to
table gathers, head products and argmaxes that a few numpy lines state
without the oracle:

- every table row that can occur is a one-hot "marker" in a column of its
  own: codec_emb row c (table 0), pred_emb[g - 1] row c (table g, g = 1..15),
  trailing row r and tts_pad each own a column;
- code-predictor head g reads the column block of table g only: its row
  f_g(c) is the marker of table g row c, so the logit of f_g(c) is the one
  positive value when the step-g input row is table g row c, and the argmax
  is f_g(c);
- the talker head reads table 15's block: its row h(c) is the marker of
  pred_emb[14] row c, so the next code 0 is h(code 15 of the last frame),
  which reaches the talker only through the 16-row sum of NextFrame (code 0
  runs through two cycles of 4 codes);
- the talker's normed state (fPastHidden) is the normalized 17-marker sum:
  its nonzero columns name the 16 codes and the trailing row (or tts_pad)
  that went into the talker's input row.

So the codes of every frame follow a closed-form chain, and a gather from the
wrong table, a head used at the wrong step or a wrong trailing row sends a
marker into a column no head reads (the argmax then falls to code 0, which no
set holds) or shows up in the decoded state.
"""
import numpy as np

from choosers import choose_code0

VOCAB, CP_VOCAB, GROUPS, HIDDEN = 3072, 2048, 16, 1024
SET = 8  # codes in use per table
TRAILING = 4  # trailing text rows of the markers frame


class Markers:
    def __init__(self, seed=5, trailing_rows=TRAILING):
        rng = np.random.default_rng(seed)
        H = HIDDEN
        # the codes in use: table 0 (codec_emb) within [1, 2048) (the talker's
        # allowed range), tables 1..15 within [1, 2048); code 0 never used
        self.sets = [np.sort(rng.choice(np.arange(1, 2048), SET, replace=False))
                     for _ in range(GROUPS)]
        col = 0
        self.col = []  # col[t][i]: the column of table t, code sets[t][i]
        for t in range(GROUPS):
            self.col.append(np.arange(col, col + SET))
            col += SET
        self.trail_col = np.arange(col, col + trailing_rows)
        col += trailing_rows
        self.pad_col = col
        col += 1
        assert col <= H
        self.trailing_rows = trailing_rows
        # f_g: table g -> table g + 1 (g = 0..14), random bijections; h: table
        # 15 -> table 0 closing an 8-cycle of code 0 over the frames
        self.f = [dict(zip(self.sets[g], rng.permutation(self.sets[g + 1])))
                  for g in range(GROUPS - 1)]
        chain = {}
        for c in self.sets[0]:
            x = c
            for g in range(GROUPS - 1):
                x = self.f[g][x]
            chain[c] = x  # code 15 of a frame whose code 0 is c
        # code 0 runs through two cycles of 4 codes (order[:4], order[4:])
        order = rng.permutation(self.sets[0])
        self.cycles = [list(order[:SET // 2]), list(order[SET // 2:])]
        nxt = {}
        for cyc in self.cycles:
            for i, c in enumerate(cyc):
                nxt[c] = cyc[(i + 1) % len(cyc)]
        self.h = {chain[c]: nxt[c] for c in self.sets[0]}
        # tables
        self.codec_emb = np.zeros((VOCAB, H), np.float32)
        self.pred_emb = [np.zeros((CP_VOCAB, H), np.float32) for _ in range(GROUPS - 1)]
        for i, c in enumerate(self.sets[0]):
            self.codec_emb[c, self.col[0][i]] = 1.0
        for g in range(1, GROUPS):
            for i, c in enumerate(self.sets[g]):
                self.pred_emb[g - 1][c, self.col[g][i]] = 1.0
        self.trailing = np.zeros((trailing_rows, H), np.float32)
        for r in range(trailing_rows):
            self.trailing[r, self.trail_col[r]] = 1.0
        self.tts_pad = np.zeros(H, np.float32)
        self.tts_pad[self.pad_col] = 1.0
        # heads
        self.cp_heads = [np.zeros((CP_VOCAB, H), np.float32) for _ in range(GROUPS - 1)]
        for g in range(GROUPS - 1):
            for i, c in enumerate(self.sets[g]):
                self.cp_heads[g][self.f[g][c], self.col[g][i]] = 1.0
        self.talker_head = np.zeros((VOCAB, H), np.float32)
        for i, c in enumerate(self.sets[GROUPS - 1]):
            self.talker_head[self.h[c], self.col[GROUPS - 1][i]] = 1.0

    def index(self, t, code):
        i = np.searchsorted(self.sets[t], code)
        assert i < SET and self.sets[t][i] == code, (t, code)
        return i

    def prefill(self, rows, start_code15):
        """rows of prompt; the last one carries the table-15 marker of
        start_code15, so the first code 0 is h(start_code15); the others are
        tts_pad markers (any row: the zero stacks ignore all but the last)."""
        p = np.zeros((rows, HIDDEN), np.float32)
        p[:, self.pad_col] = 1.0
        p[-1] = 0.0
        p[-1, self.col[GROUPS - 1][self.index(GROUPS - 1, start_code15)]] = 1.0
        return p

    def chain(self, start_code15, frames):
        """The codes of `frames` frames after a prefill from start_code15."""
        out = []
        c15 = start_code15
        for _ in range(frames):
            codes = [self.h[c15]]
            for g in range(GROUPS - 1):
                codes.append(self.f[g][codes[-1]])
            out.append(codes)
            c15 = codes[-1]
        return np.array(out, np.int64)

    def add_alternatives(self, weight=0.97):
        """A second talker-head row per table-15 marker, at `weight` (< 1):
        alt(c) = the code at the same place as h(c) in the other cycle of
        code 0. The repetition penalty then decides code 0: starting in one
        cycle, once h(c) comes round again h(c) / 1.05 < weight and the
        unseen alternative wins, moving code 0 to the other cycle; there both
        candidates have been returned and h(c) wins again."""
        a, b = self.cycles
        for i, c in enumerate(self.sets[GROUPS - 1]):
            h = self.h[c]
            alt = b[a.index(h)] if h in a else a[b.index(h)]
            self.talker_head[alt, self.col[GROUPS - 1][i]] = weight

    def add_eos(self, eos, code15, weight=1.5):
        """The talker head's eos row reads the marker of pred_emb[14] row
        code15: eos wins the code 0 after a frame ending in code15 (once two
        frames were returned; before that ChooseCode0 forbids it)."""
        self.talker_head[eos, self.col[GROUPS - 1][self.index(GROUPS - 1, code15)]] = weight

    def run(self, start_code15, frames, eos=-1, penalty=1.05):
        """The codes of up to `frames` frames after a prefill from
        start_code15, code 0 chosen by ChooseCode0 from the talker head's
        logits (its column of the table-15 marker: the normed state's other
        columns meet zero weights in every row that can win), None at eos."""
        out, history = [], []
        c15 = start_code15
        for _ in range(frames):
            lg = self.talker_head[:, self.col[GROUPS - 1][self.index(GROUPS - 1, c15)]]
            c0 = choose_code0(lg, eos, history, penalty)
            if c0 == eos:
                out.append(None)
                break
            history.append(c0)
            codes = [c0]
            for g in range(GROUPS - 1):
                codes.append(self.f[g][codes[-1]])
            out.append(np.array(codes, np.int64))
            c15 = codes[-1]
        return out

    def state_columns(self, codes, frame, trailing_rows=None):
        """The columns the talker's normed state holds after `frame` (0-based)
        with these 16 codes: one marker per table, then trailing row `frame`
        while frame < trailing_rows (the rows the stream started with, all of
        them by default), else tts_pad."""
        n = self.trailing_rows if trailing_rows is None else trailing_rows
        cols = [self.col[t][self.index(t, codes[t])] for t in range(GROUPS)]
        cols.append(self.trail_col[frame] if frame < n else self.pad_col)
        return np.sort(np.array(cols))


def zero_stack(dims):
    """Zero matrices and unit norms at dims (f32)."""
    H, hd = dims["hidden"], dims["head_dim"]
    NQ, NKV, I = dims["heads"] * hd, dims["kv_heads"] * hd, dims["intermediate"]
    layers = []
    for _ in range(dims["layers"]):
        layers.append({
            "wq": np.zeros((NQ, H), np.float32), "wk": np.zeros((NKV, H), np.float32),
            "wv": np.zeros((NKV, H), np.float32), "wo": np.zeros((H, NQ), np.float32),
            "wgate": np.zeros((I, H), np.float32), "wup": np.zeros((I, H), np.float32),
            "wdown": np.zeros((H, I), np.float32),
            "input_norm": np.ones(H, np.float32), "post_norm": np.ones(H, np.float32),
            "q_norm": np.ones(hd, np.float32), "k_norm": np.ones(hd, np.float32)})
    return layers, np.ones(H, np.float32)


def decode_state(past, tol=1e-5):
    """The nonzero columns of a normed state whose nonzeros are all equal."""
    past = np.asarray(past, np.float64)
    nz = np.flatnonzero(np.abs(past) > tol * np.abs(past).max())
    vals = past[nz]
    assert np.all(vals > 0) and vals.max() - vals.min() <= 1e-5 * vals.max(), vals
    return nz
