"""ctypes binding of the oracle (oracle/q3o.c).

TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the reference results; never by the product
path.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libq3o.so")

F32 = 0
Q8_0 = 1
BF16 = 2

_P = ctypes.c_void_p
_FP = ctypes.POINTER(ctypes.c_float)
_IP = ctypes.POINTER(ctypes.c_int)


class Config(ctypes.Structure):
    _fields_ = [
        ("layers", ctypes.c_int32), ("hidden", ctypes.c_int32), ("heads", ctypes.c_int32),
        ("kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("intermediate", ctypes.c_int32), ("rms_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float), ("dtype", ctypes.c_int32), ("kv_f16", ctypes.c_int32),
        ("act_q8", ctypes.c_int32),
    ]


class Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown",
                 "input_norm", "post_norm", "q_norm", "k_norm")]


class FrameTables(ctypes.Structure):
    _fields_ = [
        ("talker_head", ctypes.c_void_p), ("cp_heads", ctypes.c_void_p * 15),
        ("codec_emb", ctypes.c_void_p), ("pred_emb", ctypes.c_void_p * 15),
        ("vocab", ctypes.c_int32), ("cp_vocab", ctypes.c_int32), ("groups", ctypes.c_int32),
        ("eos", ctypes.c_int32), ("penalty", ctypes.c_float), ("tts_pad", ctypes.c_void_p),
    ]


class Sampling(ctypes.Structure):
    _fields_ = [
        ("do_sample", ctypes.c_int32), ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_int32), ("top_p", ctypes.c_float),
        ("sub_do_sample", ctypes.c_int32), ("sub_temperature", ctypes.c_float),
        ("sub_top_k", ctypes.c_int32), ("sub_top_p", ctypes.c_float),
        ("seed", ctypes.c_uint64),
    ]


class Trace(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("x_qkv", "y_qkv", "b_qkv", "x_o", "y_o", "b_o", "x_gu", "y_gate", "y_up",
                 "b_gu", "x_down", "y_down", "b_down")]


class CodecRes(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("a1_alpha", "a1_beta", "c1_w", "c1_b", "a2_alpha", "a2_beta", "c2_w", "c2_b")]


class CodecBlock(ctypes.Structure):
    _fields_ = [("act_alpha", ctypes.c_void_p), ("act_beta", ctypes.c_void_p),
                ("up_w", ctypes.c_void_p), ("up_b", ctypes.c_void_p), ("res", CodecRes * 3)]


class CodecWeights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p * 2) for n in
                ("up_w", "up_b", "dw_w", "dw_b", "norm_w", "norm_b", "pw1_w", "pw1_b", "pw2_w",
                 "pw2_b", "gamma")] + [
        ("conv0_w", ctypes.c_void_p), ("conv0_b", ctypes.c_void_p), ("block", CodecBlock * 4),
        ("out_alpha", ctypes.c_void_p), ("out_beta", ctypes.c_void_p),
        ("out_w", ctypes.c_void_p), ("out_b", ctypes.c_void_p)]


def codec_struct(w, cls_w=None, cls_b=None, cls_r=None):
    """(struct, keep-alive list) of the codec weight dict w (synth.codec_weights
    layout) in the q3o_codec_weights / q3h_codec_weights layout."""
    cls_w = cls_w or CodecWeights
    keep = []

    def ptr(a):
        a = np.ascontiguousarray(a, dtype=np.float32)
        keep.append(a)
        return a.ctypes.data

    s = cls_w()
    for name in ("up_w", "up_b", "dw_w", "dw_b", "norm_w", "norm_b", "pw1_w", "pw1_b", "pw2_w",
                 "pw2_b", "gamma"):
        arr = getattr(s, name)
        for i in range(2):
            arr[i] = ptr(w[name][i])
    s.conv0_w, s.conv0_b = ptr(w["conv0_w"]), ptr(w["conv0_b"])
    for i, b in enumerate(w["block"]):
        blk = s.block[i]
        blk.act_alpha, blk.act_beta = ptr(b["act_alpha"]), ptr(b["act_beta"])
        blk.up_w, blk.up_b = ptr(b["up_w"]), ptr(b["up_b"])
        for r, rw in enumerate(b["res"]):
            for k, v in rw.items():
                setattr(blk.res[r], k, ptr(v))
    s.out_alpha, s.out_beta = ptr(w["out_alpha"]), ptr(w["out_beta"])
    s.out_w, s.out_b = ptr(w["out_w"]), ptr(w["out_b"])
    return s, keep


class Codec:
    """TQwenCodec's back part (codec.pas:1040-1083) on the CPU."""

    def __init__(self, w):
        self._s, self._keep = codec_struct(w)
        self.h = lib().q3o_codec_create(ctypes.byref(self._s))

    def reset(self):
        lib().q3o_codec_reset(self.h)

    def back(self, x):
        x = _f32(x)
        frames = x.shape[0]
        pcm = np.empty(frames * 1920, dtype=np.float32)
        lib().q3o_codec_back(self.h, _fp(x), frames, _fp(pcm))
        return pcm

    def destroy(self):
        if self.h:
            lib().q3o_codec_destroy(self.h)
            self.h = None


_lib = None


def lib():
    global _lib
    if _lib is None:
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "q3o_set_threads": (None, [ctypes.c_int]),
            "q3o_get_threads": (ctypes.c_int, []),
            "q3o_fp32_to_fp16": (ctypes.c_uint16, [ctypes.c_float]),
            "q3o_fp16_to_fp32": (ctypes.c_float, [ctypes.c_uint16]),
            "q3o_fp32_to_fp16_row": (None, [_FP, _P, ctypes.c_int64]),
            "q3o_fp16_to_fp32_row": (None, [_P, _FP, ctypes.c_int64]),
            "q3o_quantize_row_q8_0": (None, [_FP, _P, ctypes.c_int64]),
            "q3o_dequantize_row_q8_0": (None, [_P, _FP, ctypes.c_int64]),
            "q3o_quantize_matrix_q8_0": (None, [_FP, _P, ctypes.c_int64, ctypes.c_int64]),
            "q3o_stack_create": (_P, [ctypes.POINTER(Config), ctypes.POINTER(Layer), _FP]),
            "q3o_stack_destroy": (None, [_P]),
            "q3o_ctx_create": (_P, [_P, ctypes.c_int]),
            "q3o_ctx_destroy": (None, [_P]),
            "q3o_ctx_reset": (None, [_P]),
            "q3o_ctx_length": (ctypes.c_int, [_P]),
            "q3o_ctx_k": (_FP, [_P, ctypes.c_int]),
            "q3o_ctx_v": (_FP, [_P, ctypes.c_int]),
            "q3o_ctx_fill": (ctypes.c_int, [_P, _FP, _FP, ctypes.c_int]),
            "q3o_rmsnorm_rows": (None, [_FP, ctypes.c_int, ctypes.c_int, _FP, ctypes.c_float,
                                        _FP]),
            "q3o_forward_embeds": (ctypes.c_int, [_P, _FP, ctypes.c_int, _FP, _FP]),
            "q3o_forward_embeds_traced": (ctypes.c_int, [_P, _FP, ctypes.c_int, _FP, _FP,
                                                         ctypes.POINTER(Trace)]),
            "q3o_head": (None, [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _FP,
                                _FP]),
            "q3o_argmax": (ctypes.c_int, [_FP, ctypes.c_int]),
            "q3o_expf": (ctypes.c_float, [ctypes.c_float]),
            "q3o_choose_code0": (ctypes.c_int, [_FP, ctypes.c_int, ctypes.c_int, _IP,
                                                ctypes.c_int, ctypes.c_float]),
            "q3o_frame_create": (_P, [_P, _P, ctypes.POINTER(FrameTables), ctypes.c_int]),
            "q3o_frame_destroy": (None, [_P]),
            "q3o_frame_start": (ctypes.c_int, [_P, _FP, ctypes.c_int, _FP, ctypes.c_int]),
            "q3o_frame_next": (ctypes.c_int, [_P, _IP]),
            "q3o_frame_logits": (_FP, [_P]),
            "q3o_frame_past_hidden": (_FP, [_P]),
            "q3o_philox4x64": (None, [ctypes.POINTER(ctypes.c_uint64),
                                      ctypes.POINTER(ctypes.c_uint64),
                                      ctypes.POINTER(ctypes.c_uint64)]),
            "q3o_draw_uniform": (ctypes.c_float, [ctypes.c_uint64, ctypes.c_uint64,
                                                  ctypes.c_uint64]),
            "q3o_sample": (ctypes.c_int, [_FP, ctypes.c_int, ctypes.c_float, ctypes.c_int,
                                          ctypes.c_float, ctypes.c_float]),
            "q3o_frame_set_sampling": (None, [_P, ctypes.POINTER(Sampling)]),
            "q3o_codec_create": (_P, [ctypes.POINTER(CodecWeights)]),
            "q3o_codec_reset": (None, [_P]),
            "q3o_codec_back": (None, [_P, _FP, ctypes.c_int, _FP]),
            "q3o_codec_destroy": (None, [_P]),
            "q3o_text_project": (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                ctypes.c_int, _FP, _FP, _FP, _FP, _IP,
                                                ctypes.c_int, _FP]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _fp(a):
    return a.ctypes.data_as(_FP) if a is not None else None


def set_threads(n):
    lib().q3o_set_threads(int(n))


def fp32_to_fp16(x):
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().q3o_fp32_to_fp16_row(_fp(x), out.ctypes.data_as(_P), x.size)
    return out


def fp16_to_fp32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().q3o_fp16_to_fp32_row(h.ctypes.data_as(_P), _fp(out), h.size)
    return out


def rmsnorm_rows(x, w, eps=1e-6):
    """The stack's RMSNorm of every row of x [rows][n] (double sums)."""
    x, w = _f32(x), _f32(w)
    x2 = x.reshape(-1, x.shape[-1])
    y = np.empty_like(x2)
    lib().q3o_rmsnorm_rows(_fp(x2), x2.shape[0], x2.shape[1], _fp(w), eps, _fp(y))
    return y.reshape(x.shape)


def quantize_q8_0(x):
    """[rows][k] float32 -> [rows][k/32*34] uint8 ggml blocks (rows in parallel)."""
    x = _f32(x)
    k = x.shape[-1]
    rows = x.size // k
    out = np.empty(x.shape[:-1] + (k // 32 * 34,), dtype=np.uint8)
    lib().q3o_quantize_matrix_q8_0(_fp(x), out.ctypes.data_as(_P), rows, k)
    return out


def dequantize_q8_0(b, k):
    b = np.ascontiguousarray(b, dtype=np.uint8)
    rows = b.size // (k // 32 * 34)
    out = np.empty((rows, k), dtype=np.float32)
    for r in range(rows):
        lib().q3o_dequantize_row_q8_0(b[r].ctypes.data_as(_P) if b.ndim > 1 else
                                      b.ctypes.data_as(_P), _fp(out[r]), k)
    return out if b.ndim > 1 else out[0]


def expf(x):
    """q3o_expf elementwise over x (float32)."""
    f = lib().q3o_expf
    return np.array([f(float(v)) for v in np.asarray(x, np.float32).ravel()],
                    np.float32).reshape(np.shape(x))


def argmax(p):
    p = _f32(p)
    return lib().q3o_argmax(_fp(p), p.size)


def choose_code0(logits, eos, history, penalty):
    lg = _f32(logits)
    h = np.ascontiguousarray(history, dtype=np.int32)
    return lib().q3o_choose_code0(_fp(lg), lg.size, eos, h.ctypes.data_as(_IP), h.size,
                                  ctypes.c_float(penalty))


def philox4x64(ctr, key):
    """Philox4x64-10 block of counter ctr (4 x uint64) under key (2 x uint64)."""
    c = (ctypes.c_uint64 * 4)(*[int(x) for x in ctr])
    k = (ctypes.c_uint64 * 2)(*[int(x) for x in key])
    o = (ctypes.c_uint64 * 4)()
    lib().q3o_philox4x64(c, k, o)
    return [int(x) for x in o]


def draw_uniform(seed, frame, group):
    return float(lib().q3o_draw_uniform(seed, frame, group))


def sample(x, temperature=1.0, top_k=0, top_p=1.0, u=0.5):
    """The library's draw from x (n <= 3072) with uniform u."""
    x = _f32(x)
    return int(lib().q3o_sample(_fp(x), x.size, temperature, top_k, top_p, u))


def text_project(emb, fc1_w, fc1_b, fc2_w, fc2_b, ids):
    """TQwenTalker.TextProject (talker.pas:390-421) over ids: float32
    [n][hidden]. emb: float32 [vocab][text_hidden], or uint16 (the BF16 bits).
    Raises IndexError for an id out of range, as the reference raises."""
    emb = np.ascontiguousarray(emb)
    dt = BF16 if emb.dtype == np.uint16 else F32
    if dt == F32:
        emb = _f32(emb)
    vocab, th = emb.shape
    fc1_w, fc1_b, fc2_w, fc2_b = _f32(fc1_w), _f32(fc1_b), _f32(fc2_w), _f32(fc2_b)
    hidden = fc2_w.shape[0]
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    y = np.empty((len(ids), hidden), dtype=np.float32)
    rc = lib().q3o_text_project(emb.ctypes.data, dt, vocab, th, hidden, _fp(fc1_w), _fp(fc1_b),
                                _fp(fc2_w), _fp(fc2_b), ids.ctypes.data_as(_IP), len(ids),
                                _fp(y))
    if rc != 0:
        raise IndexError("text token out of range")
    return y


def start_rows(project, codec_emb, ids, codec, tts_bos, tts_eos, tts_pad, codec_pad,
               codec_bos, non_streaming):
    """The rows TQwenTalker.Start (talker.pas:520-580) builds from the prompt
    ids [im_start, assistant, \\n] text [im_end, \\n, im_start, assistant, \\n]
    and the codec ids (think / language / speaker ..., codec_pad, codec_bos):
    (prefill [rows][hidden], trailing [trailing_rows][hidden]). project(ids)
    is the text projection; tts_bos / tts_eos / tts_pad are text ids, projected
    one by one as TQwenTalker.Create does (talker.pas:339-344)."""
    ids = list(ids)
    codec = list(codec)
    if len(ids) < 9:
        raise ValueError("empty text")
    ce = np.asarray(codec_emb, dtype=np.float32)
    bos, eos, pad = (project([t])[0] for t in (tts_bos, tts_eos, tts_pad))
    text = ids[3:len(ids) - 5]
    nc, nt = len(codec), len(text)
    rows = [r for r in project(ids[:3])]
    for i in range(nc - 1):
        rows.append((pad if i < nc - 2 else bos) + ce[codec[i]])
    if non_streaming:
        for r in project(text):
            rows.append(r + ce[codec_pad])
        rows.append(eos + ce[codec_pad])
        rows.append(pad + ce[codec_bos])
        trailing = [pad]
    else:
        rows.append(project(text[:1])[0] + ce[codec_bos])
        trailing = [r for r in project(text[1:])] if nt > 1 else []
        trailing.append(eos)
    return (np.stack(rows).astype(np.float32), np.stack(trailing).astype(np.float32))


class Stack:
    def __init__(self, dims, layers, final_norm, dtype, kv_f16=0, act_q8=0):
        self.dims = dict(dims)
        self.dtype = dtype
        self.act_q8 = act_q8
        self.cfg = Config(dims["layers"], dims["hidden"], dims["heads"], dims["kv_heads"],
                          dims["head_dim"], dims["intermediate"], dims["rms_eps"],
                          dims["rope_theta"], dtype, kv_f16, act_q8)
        self._keep = []
        arr = (Layer * len(layers))()
        for i, L in enumerate(layers):
            for name in Layer._fields_:
                n = name[0]
                a = np.ascontiguousarray(L[n]) if n.startswith("w") else _f32(L[n])
                self._keep.append(a)
                setattr(arr[i], n, a.ctypes.data)
        self._arr = arr
        self._final = _f32(final_norm)
        self.h = lib().q3o_stack_create(ctypes.byref(self.cfg), arr, _fp(self._final))
        if not self.h:
            raise ValueError("q3o_stack_create: invalid dimensions")

    def head(self, w, state):
        w = np.ascontiguousarray(w)
        rows = w.shape[0]
        out = np.empty(rows, dtype=np.float32)
        st = _f32(state)
        lib().q3o_head(w.ctypes.data_as(_P), self.dtype, self.act_q8, rows, self.dims["hidden"],
                       _fp(st), _fp(out))
        return out

    def destroy(self):
        if self.h:
            lib().q3o_stack_destroy(self.h)
            self.h = None


class Ctx:
    def __init__(self, stack, max_positions):
        self.stack = stack
        self.max_positions = max_positions
        self.h = lib().q3o_ctx_create(stack.h, max_positions)

    def reset(self):
        lib().q3o_ctx_reset(self.h)

    @property
    def length(self):
        return lib().q3o_ctx_length(self.h)

    def forward(self, x, layer_out=False):
        x = _f32(x)
        if x.ndim == 1:
            x = x[None, :]
        rows, H = x.shape
        normed = np.empty(H, dtype=np.float32)
        lo = np.empty((self.stack.dims["layers"], rows, H), dtype=np.float32) if layer_out \
            else None
        rc = lib().q3o_forward_embeds(self.h, _fp(x), rows, _fp(normed), _fp(lo))
        if rc:
            raise ValueError("q3o_forward_embeds: context overflow")
        return (normed, lo) if layer_out else normed

    def forward_traced(self, x):
        """forward(x) with the operands of every product: a dict of arrays
        [layers][rows][n] (x_*, y_* f32; b_* the Q8_0 blocks as uint8 rows of
        34-byte blocks, act_q8 stacks), plus "normed" (the last row's)."""
        x = _f32(x)
        if x.ndim == 1:
            x = x[None, :]
        rows, H = x.shape
        d = self.stack.dims
        Lr = (d["layers"], rows)
        NQ, NKV, I = d["heads"] * d["head_dim"], d["kv_heads"] * d["head_dim"], d["intermediate"]
        out = dict(x_qkv=np.zeros(Lr + (H,), np.float32),
                   y_qkv=np.zeros(Lr + (NQ + 2 * NKV,), np.float32),
                   x_o=np.zeros(Lr + (NQ,), np.float32), y_o=np.zeros(Lr + (H,), np.float32),
                   x_gu=np.zeros(Lr + (H,), np.float32), y_gate=np.zeros(Lr + (I,), np.float32),
                   y_up=np.zeros(Lr + (I,), np.float32), x_down=np.zeros(Lr + (I,), np.float32),
                   y_down=np.zeros(Lr + (H,), np.float32),
                   b_qkv=np.zeros(Lr + (H // 32 * 34,), np.uint8),
                   b_o=np.zeros(Lr + (NQ // 32 * 34,), np.uint8),
                   b_gu=np.zeros(Lr + (H // 32 * 34,), np.uint8),
                   b_down=np.zeros(Lr + (I // 32 * 34,), np.uint8))
        t = Trace(**{k: v.ctypes.data for k, v in out.items()})
        normed = np.empty(H, dtype=np.float32)
        lo = np.empty((d["layers"], rows, H), dtype=np.float32)
        rc = lib().q3o_forward_embeds_traced(self.h, _fp(x), rows, _fp(normed), _fp(lo),
                                             ctypes.byref(t))
        if rc:
            raise ValueError("q3o_forward_embeds: context overflow")
        out["normed"] = normed
        out["layer_out"] = lo
        return out

    def read_kv(self, layer):
        """The cache of one layer for positions [0, length): (k, v) as f32
        [kv_heads][length][head_dim] (copies; with kv_f16 the stored values
        are the half-float roundings)."""
        d = self.stack.dims
        shape = (d["kv_heads"], self.max_positions, d["head_dim"])
        n = self.length
        out = []
        for fn in (lib().q3o_ctx_k, lib().q3o_ctx_v):
            p = fn(self.h, layer)
            a = np.ctypeslib.as_array(p, shape=(int(np.prod(shape)),)).reshape(shape)
            out.append(np.array(a[:, :n, :], copy=True))
        return out[0], out[1]

    def fill(self, k, v):
        k, v = _f32(k), _f32(v)
        if lib().q3o_ctx_fill(self.h, _fp(k), _fp(v), k.shape[2]):
            raise ValueError("q3o_ctx_fill: too long")

    def destroy(self):
        if self.h:
            lib().q3o_ctx_destroy(self.h)
            self.h = None


class Frame:
    def __init__(self, talker, cp, talker_head, cp_heads, codec_emb, pred_emb, tts_pad,
                 eos=-1, penalty=1.05, max_positions=1024, groups=16):
        t = FrameTables()
        self._keep = [np.ascontiguousarray(talker_head)] + \
            [np.ascontiguousarray(h) for h in cp_heads] + [_f32(codec_emb)] + \
            [_f32(p) for p in pred_emb] + [_f32(tts_pad)]
        k = self._keep
        t.talker_head = k[0].ctypes.data
        for g in range(groups - 1):
            t.cp_heads[g] = k[1 + g].ctypes.data
            t.pred_emb[g] = k[2 + (groups - 1) + g].ctypes.data
        t.codec_emb = k[1 + (groups - 1)].ctypes.data
        t.vocab = codec_emb.shape[0]
        t.cp_vocab = pred_emb[0].shape[0]
        t.groups = groups
        t.eos = eos
        t.penalty = penalty
        t.tts_pad = k[-1].ctypes.data
        self.t = t
        self.groups = groups
        self.vocab = t.vocab
        self.hidden = codec_emb.shape[1]
        self.h = lib().q3o_frame_create(talker.h, cp.h, ctypes.byref(t), max_positions)

    def start(self, prefill, trailing=None):
        p = _f32(prefill)
        tr = _f32(trailing) if trailing is not None and len(trailing) else None
        rc = lib().q3o_frame_start(self.h, _fp(p), p.shape[0], _fp(tr),
                                   0 if tr is None else tr.shape[0])
        if rc:
            raise ValueError("q3o_frame_start failed")

    def set_sampling(self, do_sample=False, temperature=1.0, top_k=0, top_p=1.0,
                     sub_do_sample=False, sub_temperature=1.0, sub_top_k=0, sub_top_p=1.0,
                     seed=1):
        self._sampling = Sampling(int(do_sample), temperature, top_k, top_p,
                                  int(sub_do_sample), sub_temperature, sub_top_k, sub_top_p,
                                  seed)
        lib().q3o_frame_set_sampling(self.h, ctypes.byref(self._sampling))

    def next(self):
        codes = np.empty(self.groups, dtype=np.int32)
        r = lib().q3o_frame_next(self.h, codes.ctypes.data_as(_IP))
        if r < 0:
            raise ValueError("q3o_frame_next failed")
        return (codes if r == 1 else None)

    def state(self):
        lg = np.ctypeslib.as_array(lib().q3o_frame_logits(self.h), (self.vocab,)).copy()
        ph = np.ctypeslib.as_array(lib().q3o_frame_past_hidden(self.h), (self.hidden,)).copy()
        return lg, ph

    def destroy(self):
        if self.h:
            lib().q3o_frame_destroy(self.h)
            self.h = None
