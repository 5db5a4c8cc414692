"""GPU checks of the DeltaNet verify step with deferred commit (fn_gdn_verify_dev, include/faie2fn.h).

A verify call replays the kr[b] tokens of the previous call that were accepted, writes that committed state, and
runs its nt new (draft) tokens without writing state.  The reference engine family's contract for speculation is
losslessness: the verify outputs equal plain decoding bit for bit, and replay-commit leaves exactly the state plain
decoding of the accepted tokens would (reference DESIGN.md:250, 287-293).  Here:

* the new tokens' outputs equal one-token fused-block decode (fn_gdn_block_dev) of the same tokens after the
  committed prefix, bit for bit, and the float64 oracle within 1e-5;
* the committed S and the conv taps the next call reads (the last three committed raw inputs) equal the
  plain-decode state after the accepted tokens, bit for bit;
* a call with nothing to commit writes no state at all.

Every case prints what names it before the GPU calls.
"""

import numpy as np
import pytest

import fn_synth
import hiprt
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-5
NKH, NVH, DK = 16, 32, 128
SB = NVH * DK * DK * 4  # bytes of one sequence's state


def _say(*a):
    print(*a, flush=True)


class Seqs:
    """Device state of B sequences (S, conv ring, positions) plus the layer's parameters."""

    def __init__(self, lay, ring, start, rng):
        B, C = lay.B, lay.C
        self.lay, self.B, self.C, self.ring = lay, B, C, ring
        ring_h = np.zeros((B, ring, C), np.float32)
        self.hist = rng.standard_normal((B, 3, C)).astype(np.float32)  # raw inputs of positions start-3..start-1
        for b in range(B):
            for j in range(3):
                ring_h[b, (int(start[b]) - 3 + j) & (ring - 1)] = self.hist[b, j]
        self.S = hiprt.Buf.like(lay.S0)
        self.rg = hiprt.Buf.like(ring_h)
        self.pos = hiprt.Buf.like(np.asarray(start, np.int32))
        self.w, self.dt, self.sa, self.nw = (hiprt.Buf.like(x) for x in (lay.conv_w, lay.dt_bias, lay.ssm_a,
                                                                          lay.norm_w))

    def clone(self):
        c = object.__new__(Seqs)
        c.__dict__.update(self.__dict__)
        c.S, c.rg, c.pos = (hiprt.Buf(x.nbytes, x.dtype, x.shape) for x in (self.S, self.rg, self.pos))
        c.S.copy_from(self.S), c.rg.copy_from(self.rg), c.pos.copy_from(self.pos)
        return c


def decode_one(fnlib, st, b, qkv, ab, z):
    """One plain decode token of sequence b (B = 1 call on its slices); returns its output."""
    C, ring = st.C, st.ring
    dq, da, dz = hiprt.Buf.like(qkv.reshape(1, 1, C)), hiprt.Buf.like(ab.reshape(1, 1, 2 * NVH)), \
        hiprt.Buf.like(z.reshape(1, 1, NVH * DK))
    out = hiprt.Buf.empty((1, 1, NVH * DK))
    fnlib.gdn_block_dev(1, NKH, NVH, 1, ring, st.pos.ptr + 4 * b, dq.ptr, st.w.ptr, st.rg.ptr + b * ring * C * 4,
                        da.ptr, st.dt.ptr, st.sa.ptr, st.S.ptr + b * SB, dz.ptr, st.nw.ptr, out.ptr, None)
    fnlib.advance_dev(st.pos.ptr + 4 * b, 1, 1, None)
    hiprt.sync()
    return out.download()[0, 0]


def draw(lay, nt):
    st = [lay.step() for _ in range(nt)]
    return tuple(np.ascontiguousarray(np.concatenate([s[i] for s in st], axis=1)) for i in range(3))


def verify(fnlib, st, kr, rnt, rq, ra, qkv, ab, z):
    B, nt = st.B, qkv.shape[1]
    dkr = hiprt.Buf.like(np.asarray(kr, np.int32))
    dq, da, dz = hiprt.Buf.like(qkv), hiprt.Buf.like(ab), hiprt.Buf.like(z)
    out = hiprt.Buf.empty((B, nt, NVH * DK))
    fnlib.advance_by_dev(st.pos.ptr, dkr.ptr, B)
    fnlib.gdn_verify_dev(B, NKH, NVH, nt, st.ring, st.pos.ptr, dkr.ptr, rnt if rq else 0, rq.ptr if rq else None,
                         ra.ptr if ra else None, dq.ptr, st.w.ptr, st.rg.ptr, da.ptr, st.dt.ptr, st.sa.ptr, st.S.ptr,
                         dz.ptr, st.nw.ptr, out.ptr)
    hiprt.sync()
    return out.download(), (dq, da)


def test_verify_without_commit_writes_no_state(fnlib):
    _say("gdn verify kr=0, B=2, nt=4: no state written, outputs = plain decode")
    rng = np.random.default_rng(5)
    lay = fn_synth.BlockLayer(B=2, config=1, layer=21)
    st = Seqs(lay, 8, np.array([0, 7]), rng)
    S0, r0 = st.S.download(), st.rg.download()
    qkv, ab, z = draw(lay, 4)
    ref = st.clone()
    out, _ = verify(fnlib, st, [0, 0], 4, None, None, qkv, ab, z)
    assert np.array_equal(st.S.download(), S0) and np.array_equal(st.rg.download(), r0)
    assert st.pos.download().tolist() == [0, 7]
    for b in range(2):
        for t in range(4):
            o = decode_one(fnlib, ref, b, qkv[b, t], ab[b, t], z[b, t])
            assert np.array_equal(out[b, t], o), (b, t)
    # and the float64 oracle on the same tokens from the same state
    c_ref = st.hist.astype(np.float64)
    S_ref = S0.astype(np.float64)
    o_ref = oracle.gdn_block(qkv, lay.conv_w, c_ref, ab, lay.dt_bias, lay.ssm_a, S_ref, z, lay.norm_w, NKH, NVH)
    assert oracle.relerr(out, o_ref) <= TOL


@pytest.mark.parametrize("nt", [1, 4])
def test_verify_chain_matches_plain_decode(fnlib, nt):
    """Six verify steps of B = 3 sequences with random per-sequence accept counts (1..nt, and 0 once): outputs and
    committed state bit-identical to plain decode of the committed stream, and the committed state within 1e-5 of
    the float64 oracle run over that stream."""
    _say(f"gdn verify chain B=3 nt={nt} 6 steps")
    rng = np.random.default_rng(17 + nt)
    B, ring = 3, 8
    lay = fn_synth.BlockLayer(B=B, config=1, layer=22)
    start = np.array([0, 3, 77])
    st = Seqs(lay, ring, start, rng)
    ref = st.clone()                       # plain decode of the committed tokens only
    committed = [[] for _ in range(B)]     # (qkv, ab, z) of every committed token, per sequence
    kr = [0] * B
    prev = None
    for step in range(6):
        qkv, ab, z = draw(lay, nt)
        rq, ra = prev[0] if prev else (None, None)
        out, bufs = verify(fnlib, st, kr, nt, rq, ra, qkv, ab, z)
        # reference: commit the previous step's accepted tokens, then decode the new ones on a copy
        for b in range(B):
            for t in range(kr[b]):
                decode_one(fnlib, ref, b, *prev[1][b][t])
                committed[b].append(prev[1][b][t])
        assert np.array_equal(st.S.download(), ref.S.download()), step
        assert st.pos.download().tolist() == ref.pos.download().tolist()
        # the conv taps the next call reads (raw inputs of the last three committed positions); slots further back
        # may differ: plain decode writes every position's slot, a commit of kr > 3 tokens only the last three
        committed_end = st.pos.download()
        rg_v, rg_r = st.rg.download(), ref.rg.download()
        for b in range(B):
            for j in range(1, 4):
                slot = (int(committed_end[b]) - j) & (ring - 1)
                assert np.array_equal(rg_v[b, slot], rg_r[b, slot]), (step, b, j)
        trial = ref.clone()
        for b in range(B):
            for t in range(nt):
                o = decode_one(fnlib, trial, b, qkv[b, t], ab[b, t], z[b, t])
                assert np.array_equal(out[b, t], o), (step, b, t)
        toks = [[(qkv[b, t], ab[b, t], z[b, t]) for t in range(nt)] for b in range(B)]
        prev = (bufs, toks)
        kr = [int(v) for v in rng.integers(1, nt + 1, size=B)]
        if step == 3:
            kr[1] = 0                      # nothing accepted for one sequence: its state is not rewritten
    # the committed stream of sequence 0 through the float64 oracle
    S_ref = lay.S0[:1].astype(np.float64)
    c_ref = st.hist[:1].astype(np.float64)
    for q_, a_, z_ in committed[0]:
        oracle.gdn_block(q_.reshape(1, 1, -1), lay.conv_w, c_ref, a_.reshape(1, 1, -1), lay.dt_bias, lay.ssm_a, S_ref,
                         z_.reshape(1, 1, -1), lay.norm_w, NKH, NVH)
    assert oracle.relerr(st.S.download()[:1], S_ref) <= TOL


def test_verify_argument_checks(fnlib):
    _say("gdn verify argument checks")
    lay = fn_synth.BlockLayer(B=1, config=1, layer=23)
    st = Seqs(lay, 4, np.array([4]), np.random.default_rng(1))
    qkv, ab, z = draw(lay, 2)
    with pytest.raises(RuntimeError, match="ring - 3"):   # 2 committed tokens + 3 taps do not fit a ring of 4
        verify(fnlib, st, [1], 2, hiprt.Buf.like(qkv), hiprt.Buf.like(ab), qkv, ab, z)


def test_verify_kr_out_of_range_sets_status(fnlib):
    """kr[b] outside [0, rnt] is clamped into it by the kernel (it never reads past the replay rows) and recorded in the
    per-device status word as FN_STATUS_KR; an in-range call leaves the word clear."""
    import fn

    _say("gdn verify kr out of range -> status word")
    fnlib.dev_status()
    rng = np.random.default_rng(8)
    lay = fn_synth.BlockLayer(B=2, config=1, layer=25)
    st = Seqs(lay, 8, np.array([9, 12]), rng)
    rq, ra, _ = draw(lay, 4)
    qkv, ab, z = draw(lay, 2)
    out, _ = verify(fnlib, st, [2, 3], 4, hiprt.Buf.like(rq), hiprt.Buf.like(ra), qkv, ab, z)
    assert fnlib.dev_status() == 0
    out, _ = verify(fnlib, st, [6, 0], 4, hiprt.Buf.like(rq), hiprt.Buf.like(ra), qkv, ab, z)
    assert np.isfinite(out).all()
    assert fnlib.dev_status() == fn.STATUS_KR
    assert fnlib.dev_status() == 0
