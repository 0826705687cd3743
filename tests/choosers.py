"""The reference's code choosers written as its loops: ChooseCode0's logits
processors (mormot.ai.tts.qwen.talker.pas:603-629) and the first-max ArgMax
of tests/test.tts.qwen.lm.pas:109-117. Plain Python, no oracle."""
import numpy as np


def argmax(p):
    """result 0, moved to i only when p[i] > p[result]"""
    r = 0
    for i in range(1, len(p)):
        if p[i] > p[r]:
            r = i
    return r


def choose_code0(logits, eos, history, penalty):
    """-inf on [V - 1024, V) but eos, eos -inf while fewer than 2 codes were
    returned, the repetition penalty once per code of the history (s / p when
    s > 0, else s * p, skipped when the score already changed), then argmax."""
    v = np.asarray(logits, np.float32).copy()
    V = v.size
    for i in range(V - 1024, V):
        if i != eos:
            v[i] = -np.inf
    if len(history) < 2 and 0 <= eos < V:
        v[eos] = -np.inf
    if penalty != 1.0:
        for i in history:
            s = np.float32(logits[i])
            if v[i] != s:
                continue
            v[i] = np.float32(s / np.float32(penalty)) if s > 0 else np.float32(s * np.float32(penalty))
    return argmax(v)
