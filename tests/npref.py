"""An independent, vectorised numpy restatement of the verify forward.

Written from the LLaMA equations (not from the oracle's scalar loops): float64
matrix products, repeat-interleaved GQA, masked softmax over the causal rows,
rounding to the storage dtype at the same points as the device path.  It pins
the oracle's orc_verify_forward against transposed operands, wrong GQA maps,
missing RoPE or residual terms and wrong KV placement.
"""
import numpy as np

import oracle as O


def round_act(x, afmt):
    x = np.asarray(x, dtype=np.float32)
    if afmt == O.A_F16:
        return x.astype(np.float16).astype(np.float32)
    if afmt == O.A_BF16:
        return O.bf16_bits_to_f32(O.np_f32_to_bf16_bits(x)).reshape(x.shape)
    return x


def act_to_f32(a, afmt):
    if afmt == O.A_F32:
        return a.astype(np.float32)
    if afmt == O.A_F16:
        return a.view(np.float16).astype(np.float32)
    return O.bf16_bits_to_f32(a).reshape(a.shape)


def f32_to_act(x, afmt):
    if afmt == O.A_F32:
        return x.astype(np.float32)
    if afmt == O.A_F16:
        return x.astype(np.float16).view(np.uint16)
    return O.np_f32_to_bf16_bits(x).reshape(x.shape)


def embed_rows(model, tokens):
    c = model.cfg
    W = O.dequant(model.embed, c["wfmt"])
    return W[tokens].astype(np.float32)


def forward(model, pool, page_table, tokens, seq_len, rope_pairs="adjacent"):
    """pool: numpy copy of the paged cache (modified in place); returns logits [B,R,V].
    rope_pairs: "adjacent" rotates channels (2p, 2p+1) of a head (the
    reference's RoPE), "half" rotates (p, p + hd/2) (HF Llama's rotate_half),
    both with the angle pos * theta^(-2p/hd) of pair p."""
    c = model.cfg
    afmt = c["afmt"]
    B, R = tokens.shape
    h, nh, nkv, hd, ff = c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["ffn"]
    ps = pool.shape[4]
    Kp, Vp = O.kv_planes(pool)
    grp = nh // nkv
    deq = {}

    def W(lin):
        k = id(lin["w"])
        if k not in deq:
            deq[k] = O.dequant(lin, c["wfmt"])
        return deq[k]

    def rms(x, g):
        x64 = x.astype(np.float64)
        inv = 1.0 / np.sqrt((x64 * x64).sum(-1, keepdims=True) / h + np.float32(c["rms_eps"]))
        return round_act((x64 * inv * g.astype(np.float64)).astype(np.float32), afmt)

    first = slice(0, None, 2) if rope_pairs == "adjacent" else slice(0, hd // 2)
    second = slice(1, None, 2) if rope_pairs == "adjacent" else slice(hd // 2, hd)

    def rope(v, pos):
        # v [..., heads, hd]; channel first[p] pairs with second[p]
        cs = model.rope_cos[pos].astype(np.float64)
        sn = model.rope_sin[pos].astype(np.float64)
        e0 = v[..., first].astype(np.float64)
        e1 = v[..., second].astype(np.float64)
        out = np.empty_like(v)
        out[..., first] = (e0 * cs - e1 * sn).astype(np.float32)
        out[..., second] = (e0 * sn + e1 * cs).astype(np.float32)
        return out

    x = embed_rows(model, tokens.reshape(-1)).reshape(B, R, h)
    pos = seq_len[:, None] + np.arange(R)[None, :]
    for L, Ld in enumerate(model.layers):
        xn = rms(x, Ld["attn_norm"])
        qkv = (xn.astype(np.float64) @ W(Ld["qkv"]).T).astype(np.float32)
        q = qkv[..., :nh * hd].reshape(B, R, nh, hd)
        k = qkv[..., nh * hd:(nh + nkv) * hd].reshape(B, R, nkv, hd)
        v = qkv[..., (nh + nkv) * hd:].reshape(B, R, nkv, hd)
        for b in range(B):
            for j in range(R):
                q[b, j] = rope(q[b, j], pos[b, j])
                k[b, j] = rope(k[b, j], pos[b, j])
        q, k, v = round_act(q, afmt), round_act(k, afmt), round_act(v, afmt)
        for b in range(B):
            for j in range(R):
                p = pos[b, j]
                pg = page_table[b, p // ps]
                Kp[L, pg, :, p % ps] = f32_to_act(k[b, j], afmt)
                Vp[L, pg, :, p % ps] = f32_to_act(v[b, j], afmt)
        att = np.zeros((B, R, nh, hd), dtype=np.float32)
        for b in range(B):
            n = int(seq_len[b]) + R
            pages = page_table[b, :(n + ps - 1) // ps]
            Kc = act_to_f32(Kp[L, pages], afmt).transpose(1, 0, 2, 3).reshape(nkv, -1, hd)[:, :n]
            Vc = act_to_f32(Vp[L, pages], afmt).transpose(1, 0, 2, 3).reshape(nkv, -1, hd)[:, :n]
            Kq = np.repeat(Kc, grp, axis=0).astype(np.float64)
            Vq = np.repeat(Vc, grp, axis=0).astype(np.float64)
            s = np.einsum("jhd,hnd->jhn", q[b].astype(np.float64), Kq) * float(np.float32(c["attn_scale"]))
            mask = np.arange(n)[None, :] > pos[b][:, None]
            s[np.broadcast_to(mask[:, None, :], s.shape)] = -np.inf
            e = np.exp(s - s.max(-1, keepdims=True))
            att[b] = (np.einsum("jhn,hnd->jhd", e, Vq) / e.sum(-1, keepdims=True)).astype(np.float32)
        att = round_act(att.reshape(B, R, nh * hd), afmt)
        x = (x + (att.astype(np.float64) @ W(Ld["o"]).T).astype(np.float32)).astype(np.float32)
        xn = rms(x, Ld["mlp_norm"])
        gu = (xn.astype(np.float64) @ W(Ld["gate_up"]).T).astype(np.float32)
        g, u = gu[..., :ff], gu[..., ff:]
        hh = round_act(((g / (1.0 + np.exp(-g.astype(np.float64)))) * u).astype(np.float32), afmt)
        x = (x + (hh.astype(np.float64) @ W(Ld["down"]).T).astype(np.float32)).astype(np.float32)
    xn = rms(x, model.final_norm)
    return (xn.astype(np.float64) @ W(model.lm_head).T).astype(np.float32)
