"""Vectorised numpy float64 twin of the C oracle (TEST INFRASTRUCTURE ONLY).

Written separately from fn_oracle.c, with a different structure (whole-batch tensor algebra, the rotate-half form of
RoPE, an explicit convolution window), so that a slip in one restatement shows up as a disagreement between the two.
Follows the same reference lines: engine/faie2fn.cu:1366-1431 (k_gdn), :1451-1478 (k_qk_norm_rope),
:1612-1690 (k_attn_split + k_attn_combine), :2573-2576 (inv_freq).
"""

import numpy as np


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _silu(x):
    return x * _sigmoid(x)


def key_head_index(nkh, nvh, head_map):
    h = np.arange(nvh)
    return h % nkh if head_map == 0 else h // (nvh // nkh)


def gdn_core(q, k, v, beta, g, S, head_map=0):
    """q,k [B,nt,nkh,dk] normalised; v [B,nt,nvh,dv]; beta, g [B,nt,nvh]; S [B,nvh,dk,dv] float64 in place."""
    B, nt, nkh, dk = q.shape
    nvh = v.shape[2]
    kidx = key_head_index(nkh, nvh, head_map)
    outs = []
    for t in range(nt):
        qt = q[:, t, kidx].astype(np.float64)          # [B,nvh,dk]
        kt = k[:, t, kidx].astype(np.float64)
        vt = v[:, t].astype(np.float64)                # [B,nvh,dv]
        gam = np.exp(g[:, t].astype(np.float64))[..., None]   # [B,nvh,1]
        bet = beta[:, t].astype(np.float64)[..., None]
        kv = np.einsum("bhij,bhi->bhj", S, kt)
        delta = (vt - gam * kv) * bet
        S *= gam[..., None]
        S += kt[..., :, None] * delta[..., None, :]
        outs.append(np.einsum("bhij,bhi->bhj", S, qt) / np.sqrt(dk))
    return np.stack(outs, axis=1)


def gdn_block(qkv, conv_w, conv_state, ab, dt_bias, ssm_a, S, z, norm_w, nkh, nvh, dk=128, dv=128, head_map=0,
              gate_act=0, eps=1e-6):
    """Fused block; conv_state [B,3,C] float64 and S float64 updated in place; returns out [B,nt,nvh*dv]."""
    B, nt, C = qkv.shape
    w = conv_w.astype(np.float64)                      # [C,4]
    outs = []
    for t in range(nt):
        x = qkv[:, t].astype(np.float64)               # [B,C]
        win = np.concatenate([conv_state, x[:, None, :]], axis=1)   # [B,4,C] oldest first
        y = _silu(np.einsum("btc,ct->bc", win, w))
        conv_state[:] = win[:, 1:]
        q = y[:, : nkh * dk].reshape(B, nkh, dk)
        k = y[:, nkh * dk: 2 * nkh * dk].reshape(B, nkh, dk)
        v = y[:, 2 * nkh * dk:].reshape(B, nvh, dv)
        q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6)
        k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
        a = ab[:, t, :nvh].astype(np.float64) + dt_bias.astype(np.float64)
        sp = np.where(a > 20.0, a, np.log1p(np.exp(np.minimum(a, 20.0))))
        g = sp * ssm_a.astype(np.float64)
        beta = _sigmoid(ab[:, t, nvh:].astype(np.float64))
        o = gdn_core(q[:, None], k[:, None], v[:, None], beta[:, None], g[:, None], S, head_map)[:, 0]   # [B,nvh,dv]
        r = 1.0 / np.sqrt((o * o).mean(-1, keepdims=True) + eps)
        zz = z[:, t].astype(np.float64).reshape(B, nvh, dv)
        gate = _sigmoid(zz) if gate_act == 0 else _silu(zz)
        outs.append((o * r * norm_w.astype(np.float64) * gate).reshape(B, nvh * dv))
    return np.stack(outs, axis=1)


def rope_inv_freq(nrot, theta):
    i = np.arange(nrot // 2, dtype=np.float64)
    return (1.0 / theta ** (2.0 * i / nrot)).astype(np.float32)


def _norm_rope(x, w, pos, nrot, inv, eps):
    """x [..., hd] fp32, pos broadcastable to x[..., 0]; rotate-half form on the first nrot dims."""
    x = x.astype(np.float64)
    y = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w.astype(np.float64)
    ang = (np.asarray(pos, np.float32)[..., None] * inv).astype(np.float32)   # fp32 product
    cos = np.cos(ang.astype(np.float64))
    sin = np.sin(ang.astype(np.float64))
    cos = np.concatenate([cos, cos], -1)
    sin = np.concatenate([sin, sin], -1)
    rot = y[..., :nrot]
    half = nrot // 2
    rotated = np.concatenate([-rot[..., half:], rot[..., :half]], -1)
    out = y.copy()
    out[..., :nrot] = rot * cos + rotated * sin
    return out


def attn(qg, knew, vnew, wq, wk, Kc, Vc, pos, nrot=64, theta=1e7, eps=1e-6):
    """Same contract as oracle.attn; dense softmax per (b, t, head) in float64."""
    B, nt, nq, _, hd = qg.shape
    nkv = knew.shape[2]
    grp = nq // nkv
    inv = rope_inv_freq(nrot, theta)
    pos = np.asarray(pos, np.int64)
    tpos = pos[:, None] + np.arange(nt)[None, :]                        # [B,nt]
    Q = _norm_rope(qg[:, :, :, 0], wq, tpos[:, :, None], nrot, inv, eps)   # [B,nt,nq,hd]
    Kn = _norm_rope(knew, wk, tpos[:, :, None], nrot, inv, eps)          # [B,nt,nkv,hd]
    Vn = vnew.astype(np.float64)
    og = np.zeros((B, nt, nq, hd))
    for b in range(B):
        p0 = int(pos[b])
        Kall = np.concatenate([Kc[b, :p0].astype(np.float64), Kn[b]], 0)   # [p0+nt,nkv,hd]
        Vall = np.concatenate([Vc[b, :p0].astype(np.float64), Vn[b]], 0)
        for t in range(nt):
            nk = p0 + t + 1
            for g in range(nkv):
                qh = Q[b, t, g * grp:(g + 1) * grp]                       # [grp,hd]
                s = qh @ Kall[:nk, g].T / np.sqrt(hd)                      # [grp,nk]
                s -= s.max(-1, keepdims=True)
                p = np.exp(s)
                o = (p @ Vall[:nk, g]) / p.sum(-1, keepdims=True)
                gate = qg[b, t, g * grp:(g + 1) * grp, 1].astype(np.float64)
                og[b, t, g * grp:(g + 1) * grp] = o * _sigmoid(gate)
    return og, Kn, Vn


def ix_prep(iqk, wqn, wkn, IKc, BKc, pos, ixh=4, ixd=128, ixr=4, nrot=64, theta=1e7, eps=1e-6):
    """Twin of oracle.ix_prep (whole-batch numpy; same in-place contract)."""
    B, nt, _ = iqk.shape
    inv = rope_inv_freq(nrot, theta)
    tpos = np.asarray(pos, np.int64)[:, None] + np.arange(nt)[None, :]
    q = iqk[:, :, : ixh * ixd].reshape(B, nt, ixh, ixd)
    Qix = _norm_rope(q, wqn, tpos[:, :, None], nrot, inv, eps)
    for b in range(B):
        p0 = int(pos[b])
        IKc[b, p0:p0 + nt] = iqk[b, :, ixh * ixd:]
        j = np.arange(p0 // ixr, (p0 + nt) // ixr)
        if j.size:
            means = IKc[b, : (j[-1] + 1) * ixr].astype(np.float64).reshape(-1, ixr, ixd).mean(1)[j]
            BKc[b, j] = _norm_rope(means, wkn, (j * ixr)[:, None], nrot, inv, eps)
    return Qix


def ix_score(Qix, BKc, pos, max_ctx, ixr=4):
    B, nt, ixh, ixd = Qix.shape
    sc = np.zeros((B, nt, max_ctx // ixr))
    for b in range(B):
        for t in range(nt):
            nb = (int(pos[b]) + t + 1) // ixr
            dots = Qix[b, t] @ BKc[b, :nb].T                  # [ixh, nb]
            sc[b, t, :nb] = np.maximum(dots, 0.0).sum(0) / np.sqrt(ixd)
    return sc


# ------------------------------------------------------------------------------------------------------------
# GGUF weight decode, vectorised over blocks (the structure of gguf-py's quants.py: split each block into its
# fields as arrays, then whole-array float32 arithmetic in ggml's order).  Independent of quant_oracle.c, which
# walks ggml's per-row loops; both follow the reference's decoders (engine/faie2fn.cu:441-655).

IQ4_LEVELS = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)
_BLOCK = {8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210), 20: (32, 18), 21: (256, 110), 23: (256, 136),
          30: (1, 2), 16: (256, 66), 17: (256, 74), 22: (256, 82), 18: (256, 98), 42: (64, 18)}


def grid_words(name):
    """A codebook data file (csrc/<name>.inc, the one the GPU decode and the C oracle include) as uint32 words."""
    import os
    import re

    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "faie2-flashnext_amd", "csrc",
                        name + ".inc")
    text = re.sub(r"/\*.*?\*/", "", open(path).read(), flags=re.S)
    return np.array([int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", text)], np.uint32)


def iq3s_grid():
    """The IQ3_S codebook [512] uint32."""
    return grid_words("iq3s_grid")


def grid_mags(name, per):
    """Magnitudes [entries][per] of a codebook of `per` bytes per entry."""
    w = grid_words(name)
    b = ((w[:, None] >> (8 * np.arange(4, dtype=np.uint32))) & 255).reshape(-1)
    return b.reshape(-1, per).astype(np.float32)


def ksigns(idx):
    """sign bits [..., 8] of 7-bit sign indices: the index with its parity as bit 7"""
    idx = np.asarray(idx, np.int64)
    par = np.zeros_like(idx)
    for k in range(7):
        par ^= (idx >> k) & 1
    byte = idx | (par << 7)
    return (byte[..., None] >> np.arange(8)) & 1


def _le32(b):
    b = b.astype(np.uint32)
    return b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16) | (b[..., 3] << 24)


def _f16(b):
    return np.ascontiguousarray(b).view(np.float16).astype(np.float32)


def _k_scales(sc):
    """6-bit scales and mins of the 8 groups of a Q4_K / Q5_K super-block from its 12 scale bytes [n, 12]."""
    sc = sc.astype(np.uint8)
    d = np.concatenate([sc[:, 0:4] & 63, (sc[:, 8:12] & 15) | ((sc[:, 0:4] >> 6) << 4)], axis=1)
    m = np.concatenate([sc[:, 4:8] & 63, (sc[:, 8:12] >> 4) | ((sc[:, 4:8] >> 6) << 4)], axis=1)
    return d.astype(np.float32), m.astype(np.float32)


def dequant(qtype, raw, rows, cols):
    """GGUF rows -> float32 [rows, cols]."""
    qk, bb = _BLOCK[int(qtype)]
    raw = np.ascontiguousarray(raw, np.uint8).reshape(rows, cols // qk * bb)
    if qtype == 30:
        return (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(rows, cols)
    blk = raw.reshape(-1, bb)
    n = blk.shape[0]
    if qtype == 8:
        y = _f16(blk[:, :2]) * blk[:, 2:].view(np.int8).astype(np.float32)
    elif qtype == 20:
        qs = blk[:, 2:]
        y = _f16(blk[:, :2]) * IQ4_LEVELS[np.concatenate([qs & 15, qs >> 4], axis=1)]
    elif qtype == 23:
        d = _f16(blk[:, 0:2])
        sh = np.ascontiguousarray(blk[:, 2:4]).view(np.uint16).astype(np.int32)
        sl = blk[:, 4:8].astype(np.int32)
        ib = np.arange(8)
        ls = ((sl[:, ib // 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4)
        dl = d * (ls - 32).astype(np.float32)
        qs = blk[:, 8:].reshape(n, 8, 16)
        lev = IQ4_LEVELS[np.concatenate([qs & 15, qs >> 4], axis=2)]
        y = dl[:, :, None] * lev
    elif qtype in (12, 13):
        d, dmin = _f16(blk[:, 0:2]), _f16(blk[:, 2:4])
        s, m = _k_scales(blk[:, 4:16])
        qs = blk[:, 16:144] if qtype == 12 else blk[:, 48:176]
        qs = qs.reshape(n, 4, 1, 32)
        q = np.concatenate([qs & 15, qs >> 4], axis=2).reshape(n, 8, 32).astype(np.int32)
        if qtype == 13:
            qh = blk[:, 16:48].astype(np.int32)
            q = q | (((qh[:, None, :] >> np.arange(8)[None, :, None]) & 1) << 4)
        y = (d * s)[:, :, None] * q.astype(np.float32) - (dmin * m)[:, :, None]
    elif qtype == 21:
        # [n][ib][l][pair]: grid point 2l + pair of group ib; its 9-bit index takes bit 2l + pair of qh[ib]
        d = _f16(blk[:, 0:2])
        qs = blk[:, 2:66].astype(np.int64).reshape(n, 8, 4, 2)
        qh = blk[:, 66:74].astype(np.int64)
        signs = blk[:, 74:106].astype(np.int64).reshape(n, 8, 4)
        sc = blk[:, 106:110].astype(np.int64)
        ib = np.arange(8)
        scale = (sc[:, ib // 2] >> (4 * (ib % 2))) & 15
        db = d * (1 + 2 * scale).astype(np.float32)                  # [n][8], one float32 product each
        bit = 2 * np.arange(4)[:, None] + np.arange(2)[None, :]          # [l][pair]
        idx = qs | (((qh[:, :, None, None] >> bit) & 1) << 8)
        mag = (iq3s_grid()[idx][..., None] >> (8 * np.arange(4, dtype=np.uint32))) & 255  # [n][8][4][2][4]
        neg = ((signs[..., None] >> np.arange(8)) & 1).reshape(n, 8, 4, 2, 4)
        y = (db[:, :, None, None, None] * mag.astype(np.float32)) * np.where(neg == 1, -1.0, 1.0).astype(np.float32)
    elif qtype in (16, 17, 22, 18):
        d = _f16(blk[:, 0:2]).reshape(n)                                   # [n]
        f = np.float32
        if qtype == 16:   # IQ2_XXS: 4 grid bytes and a word of signs + scale per group
            q = blk[:, 2:66].reshape(n, 8, 8)
            a1 = _le32(q[:, :, 4:8])
            db = d[:, None] * (f(0.5) + (a1 >> 28).astype(f)) * f(0.25)    # [n][8]
            mags = grid_mags("iq2xxs_grid", 8)[q[:, :, 0:4].astype(np.int64)]  # [n][8][4][8]
            neg = ksigns((a1[:, :, None] >> (7 * np.arange(4))) & 127)     # [n][8][4][8]
            dbl = np.repeat(db[:, :, None], 4, axis=2)
        elif qtype == 17:  # IQ2_XS: 9-bit grid index + 7-bit sign index per 8 values, a 4-bit scale per half
            q = np.ascontiguousarray(blk[:, 2:66]).view(np.uint16).reshape(n, 8, 4).astype(np.int64)
            sc = blk[:, 66:74].astype(np.int64)
            db0 = d[:, None] * (f(0.5) + (sc & 15).astype(f)) * f(0.25)
            db1 = d[:, None] * (f(0.5) + (sc >> 4).astype(f)) * f(0.25)
            dbl = np.stack([db0, db0, db1, db1], axis=2)                   # [n][8][4]
            mags = grid_mags("iq2xs_grid", 8)[q & 511]
            neg = ksigns(q >> 9)
        elif qtype == 22:  # IQ2_S: grid low byte + 2 bits of qh, a sign byte per 8 values
            qs = blk[:, 2:34].reshape(n, 8, 4).astype(np.int64)
            sg = blk[:, 34:66].reshape(n, 8, 4).astype(np.int64)
            qh = blk[:, 66:74].astype(np.int64)
            sc = blk[:, 74:82].astype(np.int64)
            db0 = d[:, None] * (f(0.5) + (sc & 15).astype(f)) * f(0.25)
            db1 = d[:, None] * (f(0.5) + (sc >> 4).astype(f)) * f(0.25)
            dbl = np.stack([db0, db0, db1, db1], axis=2)
            e = qs | ((qh[:, :, None] << (8 - 2 * np.arange(4))) & 0x300)
            mags = grid_mags("iq2s_grid", 8)[e]
            neg = (sg[..., None] >> np.arange(8)) & 1
        else:              # IQ3_XXS: pairs of 4-magnitude grid points, a word of signs + scale per group
            qs = blk[:, 2:66].reshape(n, 8, 4, 2).astype(np.int64)
            aux = _le32(blk[:, 66:98].reshape(n, 8, 4))
            db = d[:, None] * (f(0.5) + (aux >> 28).astype(f)) * f(0.5)
            dbl = np.repeat(db[:, :, None], 4, axis=2)
            g4 = grid_mags("iq3xxs_grid", 4)
            mags = np.concatenate([g4[qs[..., 0]], g4[qs[..., 1]]], axis=-1)   # [n][8][4][8]
            neg = ksigns((aux[:, :, None] >> (7 * np.arange(4))) & 127)
        y = (dbl[..., None] * mags) * np.where(neg == 1, f(-1.0), f(1.0))
    elif qtype == 42:  # Q2_0: y = d * (q - 1)
        d = _f16(blk[:, 0:2]).reshape(n)
        q = (blk[:, 2:18, None].astype(np.int64) >> (2 * np.arange(4))) & 3   # [n][16][4] -> value 4 byte + k
        y = d[:, None] * (q.reshape(n, 64) - 1).astype(np.float32)
    elif qtype == 14:
        ql = blk[:, 0:128].reshape(n, 2, 2, 32).astype(np.int32)   # [half][first / second 32 bytes][l]
        qh = blk[:, 128:192].reshape(n, 2, 1, 32).astype(np.int32)
        sc = blk[:, 192:208].view(np.int8).reshape(n, 2, 4, 2).astype(np.float32)
        d = _f16(blk[:, 208:210]).reshape(n, 1, 1, 1)
        low = np.concatenate([ql & 15, ql >> 4], axis=2)           # quarters 0..3: bytes 0-31 lo, 32-63 lo, hi, hi
        high = (qh >> (2 * np.arange(4)).reshape(1, 1, 4, 1)) & 3
        q = (low | (high << 4)) - 32                                 # [n][half][quarter][l]
        scale = np.repeat(d * sc, 16, axis=3)                        # sc[8 half + 2 quarter + l // 16]
        y = scale * q.astype(np.float32)
    else:
        raise ValueError(f"unsupported type {qtype}")
    return np.ascontiguousarray(y, np.float32).reshape(rows, cols)
