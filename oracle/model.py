"""Float64 CPU oracle of the whole model forward (TEST INFRASTRUCTURE ONLY: the checker of fn_load / fn_forward).

A numpy restatement of the reference's forward for one sequence (engine/faie2fn.cu:2370-2450 layer_forward and
enqueue, 2463-2490 forward), on the float32 values of the weights as ggml decodes them (oracle.dequant) and the path
functions of this package (gdn_block, ix_prep / ix_score / ix_select, attn with the indexer mask).  Each piece cites
the reference kernel it restates:

* embedding: the decoded token row copied into every hyper-connection stream (k_embed, faie2fn.cu:1330-1344);
* hyper-connection read (hc_read, :2350-2359): per-stream RMSNorm (k_groupnorm, :1226-1239), the stacked down +
  inject product, t = silu(lr / HC) (k_hc_lowrank, :1266-1273), the up product, x = (1/HC) sum_s sigmoid(a_s) hn_s
  and inj_s = 2 sigmoid(inject_s / HC) (tile_mix, :873-888);
* hyper-connection write h_s += y inj_s, y for the MoE = sum_k w_k down_k + sigmoid(shared gate) shared_down
  (k_hc_add, :1281-1327);
* routing: softmax of the router logits, the top NEU by probability with ties to the lower expert, weights
  renormalized over them; the shared expert's SwiGLU (k_route, :1747-1798);
* routed experts: silu(gate_e . x) * (up_e . x) (k_tmoe_gu, :1047-1079), down_e . act (k_tmoe_down, :1159-1183);
* final read without inject, LM head, argmax with ties to the lowest index (enqueue_dev1, :2441-2447; k_argmax,
  :1910-1934);
* per-layer n-gram embedding of the layers in ple.layers, before their first read (layer_forward, :2374-2381): the
  table rows of each head from the 64-bit hash of the bigram / trigram context (k_ple_ids, :1810-1823, contexts cut
  at EOS), the key and value products of the gathered rows, the per-stream gate (k_ple_gate, :1843-1875) and the
  dilated causal conv with its 9-deep history (k_ple_conv, :1878-1896); such a layer normalizes its streams itself.

Arithmetic is float64 throughout; the path kernels' inputs pass through float32 where the GPU's do (their oracle
functions take float32 arrays), which keeps every comparison on the GPU's own input precision.
"""

import numpy as np

import oracle

HD, DS, IXH, IXD, IXR = 256, 128, 4, 128, 4


def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def _silu(x):
    return x * _sig(x)


class Model:
    """The weights of a model file (read with the GGUF reader below) and the state of one sequence."""

    def __init__(self, kv, tensors, max_ctx):
        a = kv["general.architecture"] + "."
        g = lambda k, dflt=None: kv.get(a + k, dflt)  # noqa: E731
        self.D, self.NL, self.NH, self.NKV = g("embedding_length"), g("block_count"), g("attention.head_count"), \
            g("attention.head_count_kv")
        self.NE, self.NEU, self.FFE = g("expert_count"), g("expert_used_count"), g("expert_feed_forward_length")
        self.FFS = g("expert_shared_feed_forward_length", self.FFE)
        self.NKH, self.NVH, self.HC, self.HCR = g("ssm.group_count"), g("ssm.time_step_rank"), \
            g("hyper_connection.count"), g("hyper_connection.low_rank")
        self.top = g("attention.indexer.top_k") // IXR
        self.every = g("full_attention_interval", 4)
        self.eps = float(np.float32(g("attention.layer_norm_rms_epsilon", 1e-6)))
        self.theta = float(np.float32(g("rope.freq_base", 1e7)))
        self.nrot = g("rope.dimension_count", 64)
        self.max_ctx = (max_ctx + 255) // 256 * 256
        self.t = {name: (ty, dims, raw) for name, ty, dims, raw in tensors}
        self.VOCAB = self.t["token_embd.weight"][1][1]
        self.C = 2 * self.NKH * DS + self.NVH * DS
        self.ple_layers = list(g("ple.layers", []))
        if self.ple_layers:
            self.ple_heads, self.ple_hd = 2 * g("ple.heads_per_ngram"), g("embedding_length_per_layer_input")
            self.ple_eos, self.ple_mult = g("ple.eos_token_id"), list(g("ple.layer_multipliers"))
            self.ple_off, self.ple_size = list(g("ple.head_offsets")), list(g("ple.head_vocab_sizes"))
        self._w = {}
        self.reset()

    # ---- weights ----
    def w(self, *names):
        """float64 [rows][cols] of one tensor, or of several stacked row-wise (the reference's load_qw_cat)."""
        key = names
        if key not in self._w:
            mats = []
            for n in names:
                ty, dims, raw = self.t[n]
                cols = dims[0]
                rows = int(np.prod(dims[1:])) if len(dims) > 1 else 1
                if ty == 0:
                    m = np.frombuffer(raw, np.float32).reshape(rows, cols)
                else:
                    m = oracle.dequant(ty, np.frombuffer(raw, np.uint8), rows, cols)
                mats.append(m.astype(np.float64))
            self._w[key] = mats[0] if len(mats) == 1 else np.concatenate(mats, axis=0)
        return self._w[key]

    def rows(self, name, e, R):
        """float64 rows [e R, (e + 1) R) of a tensor (one expert of a stacked expert tensor), decoded from those rows'
        bytes alone (GGUF rows are whole blocks, so a row range is a byte range)"""
        key = (name, e)
        if key not in self._w:
            ty, dims, raw = self.t[name]
            cols = dims[0]
            rb = len(raw) // int(np.prod(dims[1:]))
            part = np.frombuffer(raw, np.uint8)[e * R * rb:(e + 1) * R * rb]
            self._w[key] = oracle.dequant(ty, part, R, cols).astype(np.float64)
        return self._w[key]

    def f32(self, name):
        return np.frombuffer(self.t[name][2], np.float32).copy()

    # ---- state ----
    def reset(self):
        self.pos = 0
        self.toks = []
        self.ple_hist = {il: np.zeros((9, self.HC * self.D)) for il in self.ple_layers}
        self.S, self.conv, self.K, self.V, self.IK, self.BK = {}, {}, {}, {}, {}, {}
        for il in range(self.NL):
            if self.is_attn(il):
                self.K[il] = np.zeros((1, self.max_ctx, self.NKV, HD), np.float32)
                self.V[il] = np.zeros((1, self.max_ctx, self.NKV, HD), np.float32)
                self.IK[il] = np.zeros((1, self.max_ctx, IXD), np.float32)
                self.BK[il] = np.zeros((1, self.max_ctx // IXR, IXD), np.float64)
            else:
                self.S[il] = np.zeros((1, self.NVH, DS, DS), np.float64)
                self.conv[il] = np.zeros((1, 3, self.C), np.float64)

    def is_attn(self, il):
        return self.every > 0 and (il + 1) % self.every == 0

    # ---- pieces ----
    def groupnorm(self, h, w):
        """per-stream RMSNorm of h [nt][HC D] with weight w [HC D]"""
        nt = h.shape[0]
        hs = h.reshape(nt, self.HC, self.D)
        r = 1.0 / np.sqrt((hs * hs).mean(-1, keepdims=True) + self.eps)
        return (hs * r * w.reshape(self.HC, self.D)).reshape(nt, -1)

    def hc_read(self, hn, down, up, inj_name=None):
        """x [nt][D] and inj [nt][HC] (or None) from the normalized streams hn [nt][HC D]"""
        names = (down,) + ((inj_name,) if inj_name else ())
        lr = hn @ self.w(*names).T
        t = _silu(lr[:, : self.HCR] / self.HC)
        act = t @ self.w(up).T                                   # [nt][HC D]
        nt = hn.shape[0]
        sg = _sig(act).reshape(nt, self.HC, self.D)
        x = (sg * hn.reshape(nt, self.HC, self.D)).sum(1) / self.HC
        inj = 2.0 * _sig(lr[:, self.HCR:] / self.HC) if inj_name else None
        return x, inj

    def route(self, logits):
        """(sel [nt][NEU], w [nt][NEU]): softmax, the NEU most probable (ties: lower expert), renormalized"""
        nt = logits.shape[0]
        sel = np.zeros((nt, self.NEU), np.int64)
        wsel = np.zeros((nt, self.NEU))
        for t in range(nt):
            p = np.exp(logits[t] - logits[t].max())
            order = np.lexsort((np.arange(self.NE), -p))          # probability descending, then index ascending
            top = order[: self.NEU]
            sel[t] = top
            wsel[t] = p[top] / p[top].sum()
        return sel, wsel

    def mixer(self, il, x):
        p = f"blk.{il}."
        nt = x.shape[0]
        if not self.is_attn(il):
            qkv = x @ self.w(p + "attn_qkv.weight").T
            z = x @ self.w(p + "attn_gate.weight").T
            ab = x @ self.w(p + "ssm_alpha.weight", p + "ssm_beta.weight").T
            conv_w = self.f32(p + "ssm_conv1d.weight").reshape(self.C, 4)
            out = oracle.gdn_block(qkv[None], conv_w, self.conv[il], ab[None], self.f32(p + "ssm_dt.bias"),
                                   self.f32(p + "ssm_a"), self.S[il], z[None], self.f32(p + "ssm_norm.weight"),
                                   self.NKH, self.NVH, eps=self.eps)[0]
            return out @ self.w(p + "ssm_out.weight").T
        qg = (x @ self.w(p + "attn_q.weight").T).reshape(1, nt, self.NH, 2, HD)
        k = (x @ self.w(p + "attn_k.weight").T).reshape(1, nt, self.NKV, HD)
        v = (x @ self.w(p + "attn_v.weight").T).reshape(1, nt, self.NKV, HD)
        iqk = (x @ self.w(p + "indexer.q_proj.weight", p + "indexer.k_proj.weight").T).reshape(1, nt, -1)
        pos = np.array([self.pos], np.int32)
        Qix = oracle.ix_prep(iqk, self.f32(p + "indexer.q_norm.weight"), self.f32(p + "indexer.k_norm.weight"),
                             self.IK[il], self.BK[il], pos, nrot=self.nrot, theta=self.theta, eps=self.eps)
        sc = oracle.ix_score(Qix, self.BK[il], pos, self.max_ctx)
        mask = oracle.ix_select(sc, pos, self.top)
        og, kr, vr = oracle.attn(qg, k, v, self.f32(p + "attn_q_norm.weight"), self.f32(p + "attn_k_norm.weight"),
                                 self.K[il], self.V[il], pos, nrot=self.nrot, theta=self.theta, eps=self.eps, mask=mask,
                                 top=self.top)
        self.K[il][0, self.pos:self.pos + nt] = kr[0].astype(np.float32)
        self.V[il][0, self.pos:self.pos + nt] = vr[0].astype(np.float32)
        return og[0].reshape(nt, -1) @ self.w(p + "attn_output.weight").T

    def ffn(self, il, x):
        p = f"blk.{il}."
        nt = x.shape[0]
        rsg = x @ self.w(p + "ffn_gate_inp.weight", p + "ffn_gate_inp_shexp.weight").T
        sha = _silu(x @ self.w(p + "ffn_gate_shexp.weight").T) * (x @ self.w(p + "ffn_up_shexp.weight").T)
        shd = sha @ self.w(p + "ffn_down_shexp.weight").T
        sel, wsel = self.route(rsg[:, : self.NE])
        y = np.zeros((nt, self.D))
        for t in range(nt):
            for k in range(self.NEU):
                e = sel[t, k]
                g = self.rows(p + "ffn_gate_exps.weight", e, self.FFE) @ x[t]
                u = self.rows(p + "ffn_up_exps.weight", e, self.FFE) @ x[t]
                y[t] += wsel[t, k] * (self.rows(p + "ffn_down_exps.weight", e, self.D) @ (_silu(g) * u))
        y += _sig(rsg[:, self.NE:self.NE + 1]) * shd
        return y, sel

    # ---- per-layer n-gram embedding ----
    def ple_rows(self, p):
        """table rows of the n-gram heads at position p: mixed = t0 m0 ^ p1 m1 (^ p2 m2 for the trigram half), every
        product of the ids widened with their sign and taken modulo 2^64; row = mixed mod size + offset"""
        M = (1 << 64) - 1
        tok, eos = self.toks, self.ple_eos
        t0 = tok[p]
        p1 = tok[p - 1] if p >= 1 else eos
        p2 = tok[p - 2] if (p >= 2 and p1 != eos) else eos
        m0, m1, m2 = self.ple_mult
        rows = []
        for hd in range(self.ple_heads):
            mixed = ((t0 * m0) & M) ^ ((p1 * m1) & M)
            if hd >= self.ple_heads // 2:
                mixed ^= (p2 * m2) & M
            rows.append(mixed % self.ple_size[hd] + self.ple_off[hd])
        return rows

    def ple_gate(self, key, val, h, wk, wq, wc):
        """(gv, gvn) [nt][HC D] from key [nt][HC D], val [nt][D] and the streams h [nt][HC D]"""
        nt, HC, D = h.shape[0], self.HC, self.D
        rms = lambda x: x / np.sqrt((x * x).mean(-1, keepdims=True) + self.eps)  # noqa: E731
        kn = rms(key.reshape(nt, HC, D)) * wk.reshape(HC, D)
        qn = rms(h.reshape(nt, HC, D)) * wq.reshape(HC, D)
        gate = (kn * qn).sum(-1) / np.sqrt(D)                                       # [nt][HC]
        gate = np.where(gate == 0.0, 0.0, np.sign(gate) * np.sqrt(np.maximum(np.abs(gate), 1e-6)))
        gv = _sig(gate)[:, :, None] * val[:, None, :]
        gvn = rms(gv) * wc.reshape(HC, D)
        return gv.reshape(nt, -1), gvn.reshape(nt, -1)

    def ple_conv(self, il, gv, gvn, w):
        """h increment gv + silu(w0 x[t-9] + w1 x[t-6] + w2 x[t-3] + w3 x[t]) over x = history ++ gvn; w [HC D][4]"""
        nt = gv.shape[0]
        x = np.concatenate([self.ple_hist[il], gvn])
        out = np.zeros_like(gv)
        for t in range(nt):
            i = 9 + t
            sv = w[:, 0] * x[i - 9] + w[:, 1] * x[i - 6] + w[:, 2] * x[i - 3] + w[:, 3] * x[i]
            out[t] = gv[t] + _silu(sv)
        self.ple_hist[il] = x[nt:nt + 9].copy()
        return out

    def ple(self, il, h, nt):
        p = f"blk.{il}."
        rows = [self.ple_rows(self.pos + t) for t in range(nt)]
        table = self.ple_table()
        emb = np.stack([np.concatenate([table[r] for r in rr]) for rr in rows])      # [nt][D]
        key = emb @ self.w(p + "ple_key.weight").T
        val = emb @ self.w(p + "ple_value.weight").T
        gv, gvn = self.ple_gate(key, val, h, self.f32(p + "ple_norm_key.weight"), self.f32(p + "ple_norm_query.weight"),
                                self.f32(p + "ple_norm_conv.weight"))
        w = self.f16(p + "ple_conv1d.weight").reshape(self.HC * self.D, 4)
        return h + self.ple_conv(il, gv, gvn, w)

    def ple_table(self):
        return self.w("per_layer_token_embd.weight")

    def f16(self, name):
        ty, _, raw = self.t[name]
        return (np.frombuffer(raw, np.float16) if ty == 1 else np.frombuffer(raw, np.float32)).astype(np.float64)

    # ---- forward ----
    def forward(self, ids):
        """logits [nt][VOCAB] float64, argmax [nt], h after every layer [NL][nt][HC D], routed experts per layer"""
        ids = np.asarray(ids)
        nt = len(ids)
        self.toks[self.pos:self.pos + nt] = [int(i) for i in ids]
        emb = self.w("token_embd.weight")[ids]
        h = np.tile(emb, (1, self.HC))
        hs, sels = [], []
        for il in range(self.NL):
            p = f"blk.{il}."
            if il in self.ple_layers:
                h = self.ple(il, h, nt)
            hn = self.groupnorm(h, self.f32(p + "hc_attn_norm.weight"))
            x, inj = self.hc_read(hn, p + "hc_attn_down.weight", p + "hc_attn_up.weight", p + "hc_attn_inject.weight")
            y = self.mixer(il, x)
            h = h + (y[:, None, :] * inj[:, :, None]).reshape(nt, -1)
            hn = self.groupnorm(h, self.f32(p + "hc_ffn_norm.weight"))
            x, inj = self.hc_read(hn, p + "hc_ffn_down.weight", p + "hc_ffn_up.weight", p + "hc_ffn_inject.weight")
            y, sel = self.ffn(il, x)
            h = h + (y[:, None, :] * inj[:, :, None]).reshape(nt, -1)
            hs.append(h.copy())
            sels.append(sel)
        hn = self.groupnorm(h, self.f32("output_hc_norm.weight"))
        x, _ = self.hc_read(hn, "output_hc_down.weight", "output_hc_up.weight")
        logits = x @ self.w("output.weight").T
        am = np.array([int(np.argmax(l)) for l in logits])  # first maximum: the lowest index on ties
        self.pos += nt
        return logits, am, np.stack(hs), sels
