"""Seeded synthetic inputs of the benchmark configurations (numpy PCG64, drawn in float64, rounded to fp32 once).

The GPU path and the float64 oracle consume the identical fp32 arrays these functions return.  Draw order is
fixed and part of the contract (changing it changes every fixture):

* DeltaNet core (config 0): seed 0.  S0 ~ N(0, 0.02) [B, nvh, 128, 128]; then per step, in this order:
  q ~ N(0,1) [B, nkh, 128], k ~ N(0,1) [B, nkh, 128] (both L2-normalised in float64 with the
  x / sqrt(sum x^2 + 1e-6) form), v ~ N(0,1) [B, nvh, 128], beta = sigmoid(N(0,1)) [B, nvh],
  g = -exp(N(0, 0.5)) * softplus(N(0,1)) [B, nvh] (the two normals drawn as two [B, nvh] arrays, exp-part first).
* DeltaNet block (configs 1 and 2): seed 1000 * config + layer.  conv_w ~ N(0, 0.1) [C, 4]; A_log ~ N(0, 0.5)
  [nvh] (ssm_a = -exp(A_log)); dt_bias = 0; norm_w ~ N(1, 0.1) [128]; S0 ~ N(0, 0.02) [B, nvh, 128, 128];
  conv state zero; then per step: qkv ~ N(0,1) [B, C], z ~ N(0,1) [B, nvh*128], a ~ N(0,1) [B, nvh],
  b ~ N(0,1) [B, nvh]; ab = [a | b] per sequence.
* GQA decode (config 3): seed 3000 + ctx % 997 + 7 * B.  wq, wk ~ N(1, 0.1) [256]; cache rows
  0 .. L-2 ~ N(0,1) [B, L, nkv, 256] for K then V; q ~ N(0,1) and gate ~ N(0,1) as qg [B, 1, nq, 2, 256];
  new k, v ~ N(0,1) [B, 1, nkv, 256]; pos = L - 1.
"""

import numpy as np

DK = DV = 128
HD = 256


def _f32(x):
    return np.asarray(x, np.float64).astype(np.float32)


def _l2n(x):
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + 1e-6)


def softplus(x):
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


class CoreSteps:
    """Config 0 generator: .S0 then .step() -> (q, k, v, beta, g) with a leading nt = 1 axis."""

    def __init__(self, B=1, nkh=16, nvh=32, seed=0):
        self.B, self.nkh, self.nvh = B, nkh, nvh
        self.rng = np.random.default_rng(seed)
        self.S0 = _f32(self.rng.normal(0.0, 0.02, (B, nvh, DK, DV)))

    def step(self):
        r, B, nkh, nvh = self.rng, self.B, self.nkh, self.nvh
        q = _f32(_l2n(r.standard_normal((B, nkh, DK))))
        k = _f32(_l2n(r.standard_normal((B, nkh, DK))))
        v = _f32(r.standard_normal((B, nvh, DV)))
        beta = _f32(1.0 / (1.0 + np.exp(-r.standard_normal((B, nvh)))))
        e = r.normal(0.0, 0.5, (B, nvh))
        s = r.standard_normal((B, nvh))
        g = _f32(-np.exp(e) * softplus(s))
        return tuple(x[:, None] for x in (q, k, v, beta, g))


class BlockLayer:
    """Config 1/2 generator for one layer: parameters, S0, and .step() -> (qkv, ab, z) with nt = 1 axis."""

    def __init__(self, B=1, nkh=16, nvh=32, config=1, layer=0, seed=None):
        self.B, self.nkh, self.nvh = B, nkh, nvh
        self.C = 2 * nkh * DK + nvh * DV
        self.rng = np.random.default_rng(1000 * config + layer if seed is None else seed)
        r = self.rng
        self.conv_w = _f32(r.normal(0.0, 0.1, (self.C, 4)))
        A_log = r.normal(0.0, 0.5, nvh)
        self.ssm_a = _f32(-np.exp(A_log))
        self.dt_bias = np.zeros(nvh, np.float32)
        self.norm_w = _f32(r.normal(1.0, 0.1, DV))
        self.S0 = _f32(r.normal(0.0, 0.02, (B, nvh, DK, DV)))
        self.conv0 = np.zeros((B, 3, self.C), np.float32)

    def step(self):
        r, B, nvh = self.rng, self.B, self.nvh
        qkv = _f32(r.standard_normal((B, self.C)))
        z = _f32(r.standard_normal((B, nvh * DV)))
        a = r.standard_normal((B, nvh))
        b = r.standard_normal((B, nvh))
        ab = _f32(np.concatenate([a, b], axis=1))
        return qkv[:, None], ab[:, None], z[:, None]


class AttnCase:
    """Config 3 generator (dense GQA decode of one new token at pos = L - 1)."""

    def __init__(self, B=1, L=4096, nq=16, nkv=2, seed=None, max_ctx=None):
        self.B, self.L, self.nq, self.nkv = B, L, nq, nkv
        self.max_ctx = max_ctx or L
        r = np.random.default_rng(3000 + L % 997 + 7 * B if seed is None else seed)
        self.wq = _f32(r.normal(1.0, 0.1, HD))
        self.wk = _f32(r.normal(1.0, 0.1, HD))
        self.Kc = np.zeros((B, self.max_ctx, nkv, HD), np.float32)
        self.Vc = np.zeros((B, self.max_ctx, nkv, HD), np.float32)
        self.Kc[:, : L - 1] = r.standard_normal((B, L - 1, nkv, HD), dtype=np.float32)
        self.Vc[:, : L - 1] = r.standard_normal((B, L - 1, nkv, HD), dtype=np.float32)
        q = r.standard_normal((B, 1, nq, HD))
        gate = r.standard_normal((B, 1, nq, HD))
        self.qg = _f32(np.stack([q, gate], axis=3))
        self.k = _f32(r.standard_normal((B, 1, nkv, HD)))
        self.v = _f32(r.standard_normal((B, 1, nkv, HD)))
        self.pos = np.full(B, L - 1, np.int32)


def gdn_block_bytes(B, nkh=16, nvh=32):
    """Algorithmic HBM bytes of one fused DeltaNet layer-step for B sequences: per sequence S read + write,
    conv state read + write (3 taps of C channels), qkv, z, alpha, beta in, out; per layer conv_w, norm_w,
    dt_bias, A_log once.  = 4,588,544 at B = 1 and 285,360,896 at B = 64 for the default heads."""
    C = 2 * nkh * DK + nvh * DV
    per_seq = 2 * nvh * DK * DV * 4 + 2 * 3 * C * 4 + (C + nvh * DV + 2 * nvh) * 4 + nvh * DV * 4
    per_layer = C * 4 * 4 + DV * 4 + 2 * nvh * 4
    return B * per_seq + per_layer


def gdn_core_bytes(B, nkh=16, nvh=32):
    """Config 0 (core only): S read + write, q, k, v, beta, g in, o out."""
    return B * (2 * nvh * DK * DV * 4 + (2 * nkh * DK + 2 * nvh * DV + 2 * nvh) * 4)


def attn_bytes(B, L, nq=16, nkv=2, hd=HD, nt=1):
    """Algorithmic HBM bytes of one GQA decode layer-step: K + V read once over L keys, and per new token q, gate and
    out, new k, v (nt new tokens at positions L - nt .. L - 1 share the one K/V pass)."""
    return B * (L * nkv * hd * 4 * 2 + nt * (3 * nq * hd * 4 + 2 * nkv * hd * 4))


def attn_flops(B, L, nq=16, nkv=2, hd=HD, nt=1):
    """Algorithmic flops of the same step: q.k and p.v, 2 hd multiply-adds each, for every (query head, token, visible
    key) -- token t of nt sees L - nt + t + 1 keys."""
    keys = nt * (L - nt) + nt * (nt + 1) // 2
    return B * nq * keys * 4 * hd


def attn_qsa_bytes(B, L, top=512, nq=16, nkv=2, hd=HD, ixd=128):
    """Algorithmic HBM bytes of one sparse (QSA) decode layer-step: the block keys of the complete blocks (scored),
    K + V of the attended keys (top blocks of 4 and the tail), q, gate and out, the new k, v, the indexer input
    and its new raw key."""
    nb = L // 4
    keys = min(L, 4 * top + (L - 4 * nb)) if nb > top else L
    return B * (nb * ixd * 4 + keys * nkv * hd * 4 * 2 + 3 * nq * hd * 4 + 2 * nkv * hd * 4 + (5 * ixd + ixd) * 4)


def gdn_verify_bytes(B, nt, kr, nkh=16, nvh=32):
    """Algorithmic HBM bytes of one fused DeltaNet verify layer-step (deferred commit) for B sequences with nt new
    tokens and kr replayed (committed) tokens each: S read + write once, conv state read + write (3 taps of C
    channels), the replayed tokens' qkv and alpha/beta, the new tokens' qkv, z, alpha/beta in and outputs; per
    layer the parameters once."""
    C = 2 * nkh * DK + nvh * DV
    per_seq = (2 * nvh * DK * DV * 4 + 2 * 3 * C * 4 + kr * (C + 2 * nvh) * 4
               + nt * (C + nvh * DV + 2 * nvh) * 4 + nt * nvh * DV * 4)
    per_layer = C * 4 * 4 + DV * 4 + 2 * nvh * 4
    return B * per_seq + per_layer
