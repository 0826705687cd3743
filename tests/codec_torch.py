"""A float64 PyTorch composition of the 12 Hz decoder's back part over a whole
sequence (the modules of the reference's PyTorch model, restated with torch
operators): the independent check of the oracle's q3o_codec (test support,
imported by the codec tests only)."""
import numpy as np
import torch
import torch.nn.functional as F

RATES = (8, 5, 4, 3)
DILS = (1, 3, 9)


def _t(a):
    return torch.from_numpy(np.asarray(a, np.float64))


def causal_conv(x, w, b, dil=1):
    """x [C][T]; w [out][in][k]: conv1d with (k - 1) dil zeros on the left."""
    k = w.shape[-1]
    return F.conv1d(F.pad(x[None], ((k - 1) * dil, 0)), _t(w), _t(b), dilation=dil)[0]


def causal_tconv(x, w, b, stride):
    """ConvTranspose1d (w [in][out][k]) truncated to T stride samples."""
    T = x.shape[-1]
    return F.conv_transpose1d(x[None], _t(w), _t(b), stride=stride)[0][:, :T * stride]


def snake(x, alpha, beta):
    a = torch.exp(_t(alpha).float()).double()[:, None]
    ib = (1.0 / (torch.exp(_t(beta).float()) + 1e-9)).double()[:, None]
    return x + ib * torch.sin(x * a) ** 2


def convnext(x, w, i):
    C = x.shape[0]
    h = causal_conv_dw(x, w["dw_w"][i], w["dw_b"][i])
    h = F.layer_norm(h.T, (C,), _t(w["norm_w"][i]), _t(w["norm_b"][i]), eps=1e-6)
    h = F.gelu(F.linear(h, _t(w["pw1_w"][i]), _t(w["pw1_b"][i])))
    h = F.linear(h, _t(w["pw2_w"][i]), _t(w["pw2_b"][i]))
    return x + (_t(w["gamma"][i])[None, :] * h).T


def causal_conv_dw(x, w, b):
    C = x.shape[0]
    return F.conv1d(F.pad(x[None], (6, 0)), _t(w), _t(b), groups=C)[0]


def back(w, x, stages=None):
    """x [frames][1024] -> pcm [frames * 1920] (and the stage outputs when
    stages is a dict)."""
    h = _t(x).T  # [C][T]
    for i in range(2):
        h = causal_tconv(h, w["up_w"][i], w["up_b"][i], 2)
        h = convnext(h, w, i)
    h = causal_conv(h, w["conv0_w"], w["conv0_b"])
    if stages is not None:
        stages["conv0"] = h.T.numpy()
    for i, b in enumerate(w["block"]):
        h = snake(h, b["act_alpha"], b["act_beta"])
        h = causal_tconv(h, b["up_w"], b["up_b"], RATES[i])
        for r, rw in enumerate(b["res"]):
            c = snake(h, rw["a1_alpha"], rw["a1_beta"])
            c = causal_conv(c, rw["c1_w"], rw["c1_b"], DILS[r])
            c = snake(c, rw["a2_alpha"], rw["a2_beta"])
            c = causal_conv(c, rw["c2_w"], rw["c2_b"])
            h = h + c
        if stages is not None:
            stages[f"block{i}"] = h.T.numpy()
    h = snake(h, w["out_alpha"], w["out_beta"])
    h = causal_conv(h, w["out_w"], w["out_b"])
    if stages is not None:
        stages["out"] = h[0].numpy()
    return torch.clamp(h[0], -1.0, 1.0).numpy()
