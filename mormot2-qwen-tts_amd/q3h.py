"""ctypes binding of libq3h (include/q3h.h) and a host mirror of the reference's
stack adapter.

`QwenLm` mirrors TQwenLm of src/tts/mormot.ai.tts.qwen.lm.pas:104-143
(Create / Reset / Forward / Length); `Talker` drives the device-resident
frame step that restates TQwenTalker.Start / NextFrame
(src/tts/mormot.ai.tts.qwen.talker.pas:471-681). Errors raise Q3HError with the
library's message, as the Pascal binding raises EQwenLm (lm.pas:41).

The library must be built (see __graft_entry__.build); nothing here falls back
to a CPU path: loading fails loudly when libq3h.so is missing.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libq3h.so")

F32 = 0
Q8_0 = 1
BF16 = 2

E_ARG, E_HIP, E_CAPACITY, E_STATE, E_NODEV = -1, -2, -3, -4, -5
NOALLOC_MAX_ROWS = 64  # Q3H_NOALLOC_MAX_ROWS
NOALLOC_SCRATCH_BYTES = 16 << 20  # Q3H_NOALLOC_SCRATCH_BYTES


class Q3HError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"q3h error {code}: {msg}")
        self.code = code


class StackConfig(ctypes.Structure):
    _fields_ = [
        ("layers", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("intermediate", ctypes.c_int32),
        ("rms_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float),
        ("dtype", ctypes.c_int32),
        ("kv_f16", ctypes.c_int32),
        ("act_q8", ctypes.c_int32),
        ("max_positions", ctypes.c_int32),
    ]


class LayerWeights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown",
                 "input_norm", "post_norm", "q_norm", "k_norm")]


class Weights(ctypes.Structure):
    _fields_ = [
        ("src_dtype", ctypes.c_int32),
        ("layers", ctypes.POINTER(LayerWeights)),
        ("final_norm", ctypes.c_void_p),
    ]


class FrameConfig(ctypes.Structure):
    _fields_ = [
        ("n_streams", ctypes.c_int32),
        ("talker_head", ctypes.c_int32),
        ("cp_heads", ctypes.c_int32 * 15),
        ("vocab", ctypes.c_int32),
        ("cp_vocab", ctypes.c_int32),
        ("groups", ctypes.c_int32),
        ("eos", ctypes.c_int32),
        ("repetition_penalty", ctypes.c_float),
        ("max_frames", ctypes.c_int32),
        ("max_positions", ctypes.c_int32),
        ("use_graph", ctypes.c_int32),
    ]


class TextConfig(ctypes.Structure):
    _fields_ = [
        ("text_vocab", ctypes.c_int32),
        ("text_hidden", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("emb_dtype", ctypes.c_int32),
    ]


class Sampling(ctypes.Structure):
    _fields_ = [
        ("do_sample", ctypes.c_int32), ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_int32), ("top_p", ctypes.c_float),
        ("sub_do_sample", ctypes.c_int32), ("sub_temperature", ctypes.c_float),
        ("sub_top_k", ctypes.c_int32), ("sub_top_p", ctypes.c_float),
        ("seed", ctypes.c_uint64),
    ]


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


class StartIds(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("tts_bos", "tts_eos", "tts_pad", "codec_pad", "codec_bos")]


_P = ctypes.c_void_p
_I = ctypes.c_int
_FP = ctypes.POINTER(ctypes.c_float)
_IP = ctypes.POINTER(ctypes.c_int32)

# name -> (restype, argtypes): every entry point of include/q3h.h
SIGNATURES = {
    "q3h_device_available": (_I, []),
    "q3h_device_open": (_I, [_I, ctypes.POINTER(_P)]),
    "q3h_device_name": (ctypes.c_char_p, [_P]),
    "q3h_device_bytes": (ctypes.c_int64, [_P]),
    "q3h_device_close": (_I, [_P]),
    "q3h_last_error": (ctypes.c_char_p, []),
    "q3h_stack_create": (_I, [_P, ctypes.POINTER(StackConfig), ctypes.POINTER(Weights),
                              ctypes.POINTER(_P)]),
    "q3h_stack_add_head": (_I, [_P, _P, _I, _I, ctypes.POINTER(_I)]),
    "q3h_stack_bytes": (ctypes.c_int64, [_P]),
    "q3h_stack_destroy": (_I, [_P]),
    "q3h_context_create": (_I, [_P, _I, ctypes.POINTER(_P)]),
    "q3h_context_reset": (_I, [_P]),
    "q3h_context_length": (_I, [_P]),
    "q3h_context_destroy": (_I, [_P]),
    "q3h_context_fill_kv": (_I, [_P, _FP, _FP, _I]),
    "q3h_context_read_kv": (_I, [_P, _I, _FP, _FP]),
    "q3h_context_time_attention": (_I, [_P, _I, _FP, ctypes.POINTER(ctypes.c_int64)]),
    "q3h_forward_embeds": (_I, [_P, _FP, _I, _I, _FP, _FP]),
    "q3h_forward_embeds_noalloc": (_I, [_P, _FP, _I, _I, _FP, _FP]),
    "q3h_forward_embeds_probe": (_I, [_P, _FP, _I, _I, _FP, _FP, _FP, _FP]),
    "q3h_forward_embeds_batch": (_I, [ctypes.POINTER(_P), _I, _FP, _IP, _FP, _FP]),
    "q3h_frame_create": (_I, [_P, _P, ctypes.POINTER(FrameConfig), _FP,
                              ctypes.POINTER(_FP), _FP, ctypes.POINTER(_P)]),
    "q3h_frame_start": (_I, [_P, _I, _FP, _I, _FP, _I]),
    "q3h_frame_start_batch": (_I, [_P, _I, ctypes.POINTER(ctypes.c_int),
                                   ctypes.POINTER(_FP), ctypes.POINTER(ctypes.c_int),
                                   ctypes.POINTER(_FP), ctypes.POINTER(ctypes.c_int)]),
    "q3h_frame_step": (_I, [_P, _IP, _IP]),
    "q3h_frame_state": (_I, [_P, _I, _FP, _FP]),
    "q3h_frame_destroy": (_I, [_P]),
    "q3h_text_create": (_I, [_P, ctypes.POINTER(TextConfig), _P, _FP, _FP, _FP, _FP,
                             ctypes.POINTER(_P)]),
    "q3h_text_project": (_I, [_P, _IP, _I, _FP]),
    "q3h_text_destroy": (_I, [_P]),
    "q3h_frame_set_sampling": (_I, [_P, ctypes.POINTER(Sampling)]),
    "q3h_codec_create": (_I, [_P, ctypes.POINTER(CodecWeights), _I, ctypes.POINTER(_P)]),
    "q3h_codec_reset": (_I, [_P]),
    "q3h_codec_back": (_I, [_P, _FP, _I, _FP]),
    "q3h_codec_bytes": (ctypes.c_int64, [_P]),
    "q3h_codec_destroy": (_I, [_P]),
    "q3h_frame_start_text": (_I, [_P, _I, _P, ctypes.POINTER(StartIds), _IP, _I, _IP, _I, _I]),
    "q3h_quantize_row_q8_0": (_I, [_FP, _P, ctypes.c_int64]),
    "q3h_stack_time_gemv": (_I, [_P, _I, _I, _I, _FP, ctypes.POINTER(_I),
                                 ctypes.POINTER(ctypes.c_int64)]),
}

_lib = None


def lib():
    """The loaded libq3h (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OSError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(rc):
    if rc != 0:
        raise Q3HError(rc, lib().q3h_last_error().decode(errors="replace"))


def _fp(a):
    return a.ctypes.data_as(_FP) if a is not None else None


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def available():
    return bool(lib().q3h_device_available())


def quantize_q8_0(x):
    """ggml quantize_row_q8_0_ref of a float32 matrix [..., k]: uint8 blocks."""
    x = _f32(x)
    k = x.size
    out = np.empty(k // 32 * 34, dtype=np.uint8)
    _check(lib().q3h_quantize_row_q8_0(_fp(x), out.ctypes.data_as(_P), k))
    return out.reshape(x.shape[:-1] + (x.shape[-1] // 32 * 34,))


class Device:
    """TQwenVulkan (lm.pas:44-62) for a gfx950 device."""

    def __init__(self, ordinal=0):
        h = _P()
        _check(lib().q3h_device_open(ordinal, ctypes.byref(h)))
        self.h = h

    @property
    def name(self):
        return lib().q3h_device_name(self.h).decode()

    @property
    def bytes(self):
        return lib().q3h_device_bytes(self.h)

    def close(self):
        if self.h:
            _check(lib().q3h_device_close(self.h))
            self.h = None


class Stack:
    """A Qwen3 stack on the device (TQwen3Model.CreateStack + TQwen3Vulkan.Create)."""

    def __init__(self, dev, cfg, layers, final_norm, src_dtype):
        """cfg: dict of StackConfig fields; layers: list of dicts with wq..wdown
        (float32 [out][in] or uint8 Q8_0 blocks [out][in/32*34]) and the norm
        vectors; src_dtype: F32 or Q8_0."""
        self.cfg = dict(cfg)
        c = StackConfig(**{k: cfg[k] for k, _ in StackConfig._fields_})
        keep = []
        arr = (LayerWeights * len(layers))()
        for i, L in enumerate(layers):
            for name in ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown"):
                a = np.ascontiguousarray(L[name])
                keep.append(a)
                setattr(arr[i], name, a.ctypes.data)
            for name in ("input_norm", "post_norm", "q_norm", "k_norm"):
                a = _f32(L[name])
                keep.append(a)
                setattr(arr[i], name, a.ctypes.data)
        fn = _f32(final_norm)
        w = Weights(src_dtype, arr, fn.ctypes.data)
        h = _P()
        _check(lib().q3h_stack_create(dev.h, ctypes.byref(c), ctypes.byref(w), ctypes.byref(h)))
        self.h = h
        self.head_rows = []

    def add_head(self, w, src_dtype):
        a = np.ascontiguousarray(w)
        rows = a.shape[0]
        idx = ctypes.c_int()
        _check(lib().q3h_stack_add_head(self.h, a.ctypes.data_as(_P), rows, src_dtype,
                                        ctypes.byref(idx)))
        self.head_rows.append(rows)
        return idx.value

    @property
    def bytes(self):
        return lib().q3h_stack_bytes(self.h)

    def time_gemv(self, head=-1, iters=20, mode=1):
        """(us per launch, launches per step, algorithmic bytes per step) of the
        weight products of one single-row decode step. mode 0: direct launches,
        wall time; 1: hipGraph replay, wall time; 2: the kernels' own execution
        time (events attached to each launch)."""
        us = ctypes.c_float()
        n = ctypes.c_int()
        b = ctypes.c_int64()
        _check(lib().q3h_stack_time_gemv(self.h, head, iters, int(mode), ctypes.byref(us),
                                         ctypes.byref(n), ctypes.byref(b)))
        return us.value, n.value, b.value

    def destroy(self):
        if self.h:
            _check(lib().q3h_stack_destroy(self.h))
            self.h = None


class Context:
    """A K/V cache of a stack (NewContext / TDecoderContext)."""

    def __init__(self, stack, max_positions):
        h = _P()
        _check(lib().q3h_context_create(stack.h, max_positions, ctypes.byref(h)))
        self.h = h
        self.stack = stack

    def reset(self):
        _check(lib().q3h_context_reset(self.h))

    @property
    def length(self):
        n = lib().q3h_context_length(self.h)
        if n < 0:
            _check(n)
        return n

    def forward(self, x, head=-1, want_logits=True, want_normed=True, noalloc=False):
        """x [rows][hidden]; returns (logits or None, normed_last or None).
        noalloc: through q3h_forward_embeds_noalloc (work buffers in the
        device's static scratch array, at most NOALLOC_MAX_ROWS rows)."""
        x = _f32(x)
        if x.ndim == 1:
            x = x[None, :]
        rows, hidden = x.shape
        logits = None
        if 0 <= head < len(self.stack.head_rows) and want_logits:
            logits = np.empty(self.stack.head_rows[head], dtype=np.float32)
        normed = np.empty(hidden, dtype=np.float32) if want_normed else None
        # an unknown head index goes to the library, which reports it
        fn = lib().q3h_forward_embeds_noalloc if noalloc else lib().q3h_forward_embeds
        _check(fn(self.h, _fp(x), rows, head, _fp(logits), _fp(normed)))
        return logits, normed

    def forward_probe(self, x, head=-1):
        """forward() with the probe of TQwenLm (lm.pas:380-389): returns
        (logits or None, normed_last, layer_out [layers][rows][hidden],
        normed_rows [rows][hidden]): every layer's output ("name.layerN") and
        the final-normed state of every row ("name.out")."""
        x = _f32(x)
        if x.ndim == 1:
            x = x[None, :]
        rows, hidden = x.shape
        logits = None
        if 0 <= head < len(self.stack.head_rows):
            logits = np.empty(self.stack.head_rows[head], dtype=np.float32)
        normed = np.empty(hidden, dtype=np.float32)
        lo = np.empty((self.stack.cfg["layers"], rows, hidden), dtype=np.float32)
        nr = np.empty((rows, hidden), dtype=np.float32)
        _check(lib().q3h_forward_embeds_probe(self.h, _fp(x), rows, head, _fp(logits),
                                              _fp(normed), _fp(lo), _fp(nr)))
        return logits, normed, lo, nr

    def fill_kv(self, k, v):
        """k, v: float32 [layers][kv_heads][len][head_dim]."""
        k, v = _f32(k), _f32(v)
        _check(lib().q3h_context_fill_kv(self.h, _fp(k), _fp(v), k.shape[2]))

    def time_attention(self, iters=20):
        """(us per launch, algorithmic bytes per launch) of the decode attention
        of one new row at position length, averaged over the layers and iters
        (events attached to each launch); the length does not change."""
        us = ctypes.c_float()
        b = ctypes.c_int64()
        _check(lib().q3h_context_time_attention(self.h, iters, ctypes.byref(us), ctypes.byref(b)))
        return us.value, b.value

    def read_kv(self, layer):
        c = self.stack.cfg
        n = self.length
        k = np.empty((c["kv_heads"], n, c["head_dim"]), dtype=np.float32)
        v = np.empty_like(k)
        _check(lib().q3h_context_read_kv(self.h, layer, _fp(k), _fp(v)))
        return k, v

    def destroy(self):
        if self.h:
            _check(lib().q3h_context_destroy(self.h))
            self.h = None


def forward_batch(ctxs, x, heads=None, want_normed=True):
    """One row per context: x [n][hidden]; heads: list of head indices or None."""
    x = _f32(x)
    n, hidden = x.shape
    arr = (_P * n)(*[c.h.value for c in ctxs])
    logits = None
    hp = None
    if heads is not None:
        ha = np.ascontiguousarray(heads, dtype=np.int32)
        hp = ha.ctypes.data_as(_IP)
        logits = np.empty((n, ctxs[0].stack.head_rows[heads[0]]), dtype=np.float32)
    normed = np.empty((n, hidden), dtype=np.float32) if want_normed else None
    _check(lib().q3h_forward_embeds_batch(arr, n, _fp(x), hp, _fp(logits), _fp(normed)))
    return logits, normed


class QwenLm:
    """TQwenLm (lm.pas:104-143): one stack, its heads, one context.

    forward(x, rows, output) follows TQwenLm.Forward (lm.pas:391-408): the rows
    are appended at positions length..length+rows-1, the normed state of the
    last row and the logits of head `output` come back."""

    def __init__(self, stack, max_positions):
        self.stack = stack
        self.ctx = Context(stack, max_positions)
        self.length = 0

    def reset(self):
        self.ctx.reset()
        self.length = 0

    def forward(self, x, output=-1):
        x = _f32(x)
        rows = 1 if x.ndim == 1 else x.shape[0]
        if rows <= 0:
            return None, None
        logits, hidden = self.ctx.forward(x, output)
        self.length += rows
        return logits, hidden

    def destroy(self):
        self.ctx.destroy()


class TextProj:
    """The talker's text projection on the device (TQwenTalker.TextProject,
    talker.pas:390-421): emb float32 [vocab][text_hidden] or uint16 (the BF16
    bits), fc1 [text_hidden][text_hidden], fc2 [hidden][text_hidden] + biases."""

    def __init__(self, dev, emb, fc1_w, fc1_b, fc2_w, fc2_b):
        emb = np.ascontiguousarray(emb)
        dt = BF16 if emb.dtype == np.uint16 else F32
        if dt == F32:
            emb = _f32(emb)
        self._w = [_f32(fc1_w), _f32(fc1_b), _f32(fc2_w), _f32(fc2_b)]
        cfg = TextConfig(emb.shape[0], emb.shape[1], self._w[2].shape[0], dt)
        h = _P()
        _check(lib().q3h_text_create(dev.h, ctypes.byref(cfg), emb.ctypes.data_as(_P),
                                     *[_fp(a) for a in self._w], ctypes.byref(h)))
        self._w = None
        self.h = h
        self.hidden = cfg.hidden

    def project(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        y = np.empty((len(ids), self.hidden), dtype=np.float32)
        _check(lib().q3h_text_project(self.h, ids.ctypes.data_as(_IP), len(ids), _fp(y)))
        return y

    def destroy(self):
        if self.h:
            _check(lib().q3h_text_destroy(self.h))
            self.h = None


class Codec:
    """The back part of the 12 Hz decoder on the device (TQwenCodecVulkan:
    Back / Reset, codec.vulkan.pas:455-488, 633-652). w: dict of the
    decoder.* tensors (f32, safetensors layouts; see synth.codec_weights)."""

    def __init__(self, dev, w, max_frames=16):
        keep = []

        def ptr(a):
            if a is None:
                return None  # NULL: the library reports the missing tensor
            a = np.ascontiguousarray(a, dtype=np.float32)
            keep.append(a)
            return a.ctypes.data

        s = CodecWeights()
        for name in ("up_w", "up_b", "dw_w", "dw_b", "norm_w", "norm_b", "pw1_w", "pw1_b",
                     "pw2_w", "pw2_b", "gamma"):
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
        h = _P()
        _check(lib().q3h_codec_create(dev.h, ctypes.byref(s), max_frames, ctypes.byref(h)))
        self.h = h

    def back(self, x):
        """x [frames][1024] -> pcm [frames * 1920]."""
        x = _f32(x)
        frames = x.shape[0]
        pcm = np.empty(frames * 1920, dtype=np.float32)
        _check(lib().q3h_codec_back(self.h, _fp(x), frames, _fp(pcm)))
        return pcm

    def reset(self):
        _check(lib().q3h_codec_reset(self.h))

    @property
    def bytes(self):
        return lib().q3h_codec_bytes(self.h)

    def destroy(self):
        if self.h:
            _check(lib().q3h_codec_destroy(self.h))
            self.h = None


class Frame:
    """The device-resident frame step over n streams (q3h_frame_*)."""

    def __init__(self, talker, cp, codec_emb, pred_emb, tts_pad, n_streams=1, talker_head=0,
                 cp_heads=None, eos=-1, penalty=1.05, max_frames=256, max_positions=1024,
                 use_graph=True, groups=16):
        vocab, hidden = codec_emb.shape
        cp_vocab = pred_emb[0].shape[0]
        cfg = FrameConfig()
        cfg.n_streams = n_streams
        cfg.talker_head = talker_head
        heads = list(cp_heads) if cp_heads is not None else list(range(groups - 1))
        for i in range(15):
            cfg.cp_heads[i] = heads[i] if i < len(heads) else 0
        cfg.vocab = vocab
        cfg.cp_vocab = cp_vocab
        cfg.groups = groups
        cfg.eos = eos
        cfg.repetition_penalty = penalty
        cfg.max_frames = max_frames
        cfg.max_positions = max_positions
        cfg.use_graph = 1 if use_graph else 0
        self.cfg = cfg
        ce = _f32(codec_emb)
        pe = [_f32(p) for p in pred_emb]
        pa = (_FP * len(pe))(*[_fp(p) for p in pe])
        tp = _f32(tts_pad)
        h = _P()
        _check(lib().q3h_frame_create(talker.h, cp.h, ctypes.byref(cfg), _fp(ce), pa, _fp(tp),
                                      ctypes.byref(h)))
        self.h = h
        self.n = n_streams
        self.groups = groups
        self.vocab = vocab
        self.hidden = hidden

    def start(self, stream, prefill, trailing=None):
        p = _f32(prefill)
        t = _f32(trailing) if trailing is not None and len(trailing) else None
        _check(lib().q3h_frame_start(self.h, stream, _fp(p), p.shape[0], _fp(t),
                                     0 if t is None else t.shape[0]))

    def start_batch(self, streams, prefills, trailings=None):
        """q3h_frame_start_batch: the starts of several streams at once, their
        prefills overlapping on the device (prefills[i] [rows][hidden],
        trailings[i] None or [rows][hidden])."""
        n = len(streams)
        ps = [_f32(p) for p in prefills]
        ts = [None] * n if trailings is None else \
            [_f32(t) if t is not None and len(t) else None for t in trailings]
        c_streams = (ctypes.c_int * n)(*[int(x) for x in streams])
        c_pre = (_FP * n)(*[_fp(p) for p in ps])
        c_rows = (ctypes.c_int * n)(*[p.shape[0] for p in ps])
        c_tr = (_FP * n)(*[_fp(t) for t in ts])
        c_trr = (ctypes.c_int * n)(*[0 if t is None else t.shape[0] for t in ts])
        _check(lib().q3h_frame_start_batch(self.h, n, c_streams, c_pre, c_rows, c_tr, c_trr))

    def set_sampling(self, do_sample=False, temperature=1.0, top_k=0, top_p=1.0,
                     sub_do_sample=False, sub_temperature=1.0, sub_top_k=0, sub_top_p=1.0,
                     seed=0):
        """TQwenTalker.Sampling (talker.pas:150): the talker's and the code
        predictor's choosers; seed 0 draws a fresh sentence seed per start."""
        sp = Sampling(int(do_sample), temperature, top_k, top_p, int(sub_do_sample),
                      sub_temperature, sub_top_k, sub_top_p, seed)
        _check(lib().q3h_frame_set_sampling(self.h, ctypes.byref(sp)))

    def start_text(self, stream, proj, ids, codec, tts_bos, tts_eos, tts_pad, codec_pad,
                   codec_bos, non_streaming):
        """TQwenTalker.Start from token ids (talker.pas:471-593): the prefill
        and trailing rows built on the device with proj (a TextProj)."""
        sp = StartIds(tts_bos, tts_eos, tts_pad, codec_pad, codec_bos)
        a = np.ascontiguousarray(ids, dtype=np.int32)
        c = np.ascontiguousarray(codec, dtype=np.int32)
        _check(lib().q3h_frame_start_text(self.h, stream, proj.h, ctypes.byref(sp),
                                          a.ctypes.data_as(_IP), len(a),
                                          c.ctypes.data_as(_IP), len(c),
                                          1 if non_streaming else 0))

    def step(self):
        codes = np.empty((self.n, self.groups), dtype=np.int32)
        alive = np.empty(self.n, dtype=np.int32)
        _check(lib().q3h_frame_step(self.h, codes.ctypes.data_as(_IP),
                                    alive.ctypes.data_as(_IP)))
        return codes, alive

    def state(self, stream):
        logits = np.empty(self.vocab, dtype=np.float32)
        past = np.empty(self.hidden, dtype=np.float32)
        _check(lib().q3h_frame_state(self.h, stream, _fp(logits), _fp(past)))
        return logits, past

    def destroy(self):
        if self.h:
            _check(lib().q3h_frame_destroy(self.h))
            self.h = None
