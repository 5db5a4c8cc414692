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
  :1910-1934).

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
            self._w[key] = np.concatenate(mats, axis=0)
        return self._w[key]

    def f32(self, name):
        return np.frombuffer(self.t[name][2], np.float32).copy()

    # ---- state ----
    def reset(self):
        self.pos = 0
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
        Wg, Wu, Wd = self.w(p + "ffn_gate_exps.weight"), self.w(p + "ffn_up_exps.weight"), \
            self.w(p + "ffn_down_exps.weight")
        y = np.zeros((nt, self.D))
        for t in range(nt):
            for k in range(self.NEU):
                e = sel[t, k]
                g = Wg[e * self.FFE:(e + 1) * self.FFE] @ x[t]
                u = Wu[e * self.FFE:(e + 1) * self.FFE] @ x[t]
                y[t] += wsel[t, k] * (Wd[e * self.D:(e + 1) * self.D] @ (_silu(g) * u))
        y += _sig(rsg[:, self.NE:self.NE + 1]) * shd
        return y, sel

    # ---- forward ----
    def forward(self, ids):
        """logits [nt][VOCAB] float64, argmax [nt], h after every layer [NL][nt][HC D], routed experts per layer"""
        ids = np.asarray(ids)
        nt = len(ids)
        emb = self.w("token_embd.weight")[ids]
        h = np.tile(emb, (1, self.HC))
        hs, sels = [], []
        for il in range(self.NL):
            p = f"blk.{il}."
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
