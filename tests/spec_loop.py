"""A greedy speculative-decoding driver shared by the oracle and the GPU tests.

`step(model_key, tokens[1][R], ctx) -> logits[1][R][V]` runs one verify
forward over R rows at positions ctx..ctx+R-1 of a single sequence, writing
their K/V.  The driver keeps target and draft caches consistent the way an
engine does: after a verify step that accepted n of K drafts the target cache
is valid up to ctx+n (inclusive) and the draft model re-consumes whatever it
has not seen yet.
"""
import numpy as np


def greedy(step, prompt, n_new):
    lg = step("t", np.array([prompt], np.int32), 0)
    nxt = int(np.argmax(lg[0, -1]))
    ctx, out, gaps = len(prompt), [], []
    while len(out) < n_new:
        out.append(nxt)
        lg = step("t", np.array([[nxt]], np.int32), ctx)
        ctx += 1
        s = np.sort(lg[0, 0].astype(np.float64))
        gaps.append(s[-1] - s[-2])
        nxt = int(np.argmax(lg[0, 0]))
    return out[:n_new], gaps


def speculative(step, accept, prompt, n_new, K):
    lg = step("t", np.array([prompt], np.int32), 0)
    step("d", np.array([prompt], np.int32), 0)
    nxt = int(np.argmax(lg[0, -1]))
    ctx = dctx = len(prompt)
    pending = [nxt]
    out, hist = [], []
    while len(out) < n_new:
        drafts = []
        dl = step("d", np.array([pending], np.int32), dctx)
        dctx += len(pending)
        d = int(np.argmax(dl[0, -1]))
        drafts.append(d)
        for _ in range(K - 1):
            dl = step("d", np.array([[d]], np.int32), dctx)
            dctx += 1
            d = int(np.argmax(dl[0, 0]))
            drafts.append(d)
        toks, n = accept(np.array([[nxt] + drafts], np.int32), ctx)
        hist.append(n)
        out.extend([nxt] + [int(t) for t in toks[:n]])
        ctx += n + 1
        nxt = int(toks[n])
        if n == K:
            pending = [drafts[-1], nxt]
        else:
            dctx = ctx
            pending = [nxt]
    return out[:n_new], hist
