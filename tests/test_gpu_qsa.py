"""GPU parity of the QSA sparse attention (indexer + selection + attention over the kept keys).

Checked separately, so that an exact selection rule is held to an exact standard:
* scores against the float64 oracle (normwise <= 1e-5 over the complete blocks of each sparse query);
* the kept-block set bit-exactly against the selection rule applied to the GPU's own scores (top blocks, ties at
  the threshold lowest index first); against the oracle's float64 scores the sets may differ only at near-ties;
* the attention output against the oracle's masked attention under the GPU's selection (<= 1e-5), and the
  appended K, V and raw index-key rows.
"""

import numpy as np
import pytest

import hiprt
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _say(*a):
    print(*a, flush=True)


def make_case(B, nt, max_ctx, pos, seed, nq=16, nkv=2, hd=256):
    rng = np.random.default_rng(seed)
    pos = np.asarray(pos, np.int32)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    c = dict(qg=f(B, nt, nq, 2, hd), k=f(B, nt, nkv, hd), v=f(B, nt, nkv, hd), iqk=f(B, nt, 640),
             wq=rng.normal(1, 0.1, hd).astype(np.float32), wk=rng.normal(1, 0.1, hd).astype(np.float32),
             wqn=rng.normal(1, 0.1, 128).astype(np.float32), wkn=rng.normal(1, 0.1, 128).astype(np.float32),
             Kc=np.zeros((B, max_ctx, nkv, hd), np.float32), Vc=np.zeros((B, max_ctx, nkv, hd), np.float32),
             IKc=np.zeros((B, max_ctx, 128), np.float32), pos=pos)
    for b in range(B):
        n = int(pos[b])
        c["Kc"][b, :n] = f(n, nkv, hd)
        c["Vc"][b, :n] = f(n, nkv, hd)
        c["IKc"][b, :n] = f(n, 128)
    return c


def run_and_check(fnlib, c, top):
    B, nt = c["qg"].shape[:2]
    max_ctx = c["Kc"].shape[1]
    Kc, Vc, IKc = c["Kc"].copy(), c["Vc"].copy(), c["IKc"].copy()
    og, sc, mask = fnlib.attn_qsa(c["qg"], c["k"], c["v"], c["wq"], c["wk"], Kc, Vc, c["iqk"], c["wqn"], c["wkn"], IKc,
                                  c["pos"], top=top)
    # oracle indexer on the same inputs
    IK_ref = c["IKc"].copy()
    BK_ref = np.zeros((B, max_ctx // 4, 128))
    for b in range(B):
        oracle.ix_blocks(IK_ref[b:b + 1], c["wkn"], BK_ref[b:b + 1], 0, int(c["pos"][b]) // 4)
    Qix = oracle.ix_prep(c["iqk"], c["wqn"], c["wkn"], IK_ref, BK_ref, c["pos"])
    sref = oracle.ix_score(Qix, BK_ref, c["pos"], max_ctx)
    sparse = 0
    for b in range(B):
        for t in range(nt):
            nb = (int(c["pos"][b]) + t + 1) // 4
            if nb <= top:
                assert not mask[b, t].any()
                continue
            sparse += 1
            assert oracle.relerr(sc[b, t, :nb], sref[b, t, :nb]) <= TOL, (b, t)
            # the selection rule, exactly, on the GPU's own scores
            want = oracle.ix_select(sc[b:b + 1, t:t + 1].astype(np.float64), np.array([int(c["pos"][b]) + t]), top)
            assert np.array_equal(mask[b, t], want[0, 0]), (b, t)
            assert int(mask[b, t].sum()) == top
            # against the float64 selection: only near-ties at the threshold may differ
            ref_mask = oracle.ix_select(sref[b:b + 1, t:t + 1], np.array([int(c["pos"][b]) + t]), top)[0, 0]
            diff = np.nonzero(ref_mask[:nb] != mask[b, t, :nb])[0]
            if diff.size:
                thr = np.sort(sref[b, t, :nb])[::-1][top - 1]
                assert np.all(np.abs(sref[b, t, diff] - thr) <= 1e-5 * np.abs(sref[b, t, :nb]).max()), (b, t, diff)
    # attention under the GPU's selection
    ref_og, ref_k, ref_v = oracle.attn(c["qg"], c["k"], c["v"], c["wq"], c["wk"], c["Kc"], c["Vc"], c["pos"],
                                       mask=mask, ixr=4, top=top)
    got_k = np.stack([Kc[b, c["pos"][b]:c["pos"][b] + nt] for b in range(B)])
    got_v = np.stack([Vc[b, c["pos"][b]:c["pos"][b] + nt] for b in range(B)])
    got_ik = np.stack([IKc[b, c["pos"][b]:c["pos"][b] + nt] for b in range(B)])
    e = (oracle.relerr(og, ref_og), oracle.relerr(got_k, ref_k), oracle.relerr(got_v, ref_v))
    assert max(e) <= TOL, e
    assert np.array_equal(got_ik, c["iqk"][:, :, 512:])
    return sparse


def test_qsa_sparse_and_dense_queries_in_one_batch(fnlib):
    """top = 64 over up to 700 keys: sequence 0 sparse (nb 174 > 64), sequence 1 dense (nb 40), sequence 2 right at
    the switch (nb 65)."""
    _say("qsa B=3 top=64 mixed sparse/dense")
    c = make_case(3, 1, 768, [699, 160, 260], seed=1)
    assert run_and_check(fnlib, c, top=64) == 2


def test_qsa_reference_budget(fnlib):
    """The reference's budget: top 512 blocks of 4 (2048 keys) at a 3000-key context."""
    _say("qsa B=1 L=3000 top=512")
    c = make_case(1, 1, 3072, [2999], seed=2)
    assert run_and_check(fnlib, c, top=512) == 1


def test_qsa_multi_token_blocks_complete_inside_the_call(fnlib):
    """nt = 5: blocks completed by this call's own new keys are built and scored (token t sees blocks
    < (pos + t + 1) / 4)."""
    _say("qsa nt=5 top=32")
    c = make_case(2, 5, 512, [301, 255], seed=3)
    run_and_check(fnlib, c, top=32)


def test_qsa_ties_keep_lowest_index(fnlib):
    """Identical raw keys make identical block scores everywhere: the kept blocks must be the lowest-index ones."""
    _say("qsa ties")
    c = make_case(1, 1, 1024, [999], seed=4)
    c["IKc"][0, :999] = c["IKc"][0, 0]  # every complete block has the same mean ... but a RoPE'd key per position
    Kc, Vc, IKc = c["Kc"].copy(), c["Vc"].copy(), c["IKc"].copy()
    og, sc, mask = fnlib.attn_qsa(c["qg"], c["k"], c["v"], c["wq"], c["wk"], Kc, Vc, c["iqk"], c["wqn"], c["wkn"], IKc,
                                  c["pos"], top=32)
    nb = 1000 // 4
    want = oracle.ix_select(sc.astype(np.float64), c["pos"], 32)
    assert np.array_equal(mask, want)
    # force exact ties: zero index queries give all-zero scores (relu of 0), so the first 32 blocks are kept
    c["iqk"][:, :, :512] = 0
    Kc, Vc, IKc = c["Kc"].copy(), c["Vc"].copy(), c["IKc"].copy()
    og, sc, mask = fnlib.attn_qsa(c["qg"], c["k"], c["v"], c["wq"], c["wk"], Kc, Vc, c["iqk"], c["wqn"], c["wkn"], IKc,
                                  c["pos"], top=32)
    assert not sc[0, 0, :nb].any()
    assert mask[0, 0, :32].all() and not mask[0, 0, 32:].any()


@pytest.mark.parametrize("nb", [600, 2000, 7000])
def test_qsa_mass_ties_fall_back_to_radix(fnlib, nb):
    """All-zero scores (zero index queries) put every complete block in one histogram bin: 600 blocks are ranked in
    the LDS by index; 2000 and 7000 exceed the 1024 the one-pass selection ranks and take the radix passes.  Either
    way the first `top` blocks are kept."""
    top = 512
    pos = nb * 4 + 1
    max_ctx = (pos + 256) // 256 * 256
    _say(f"qsa mass ties nb={nb} top={top}")
    c = make_case(1, 1, max_ctx, [pos], seed=6)
    c["iqk"][:, :, :512] = 0
    Kc, Vc, IKc = c["Kc"].copy(), c["Vc"].copy(), c["IKc"].copy()
    og, sc, mask = fnlib.attn_qsa(c["qg"], c["k"], c["v"], c["wq"], c["wk"], Kc, Vc, c["iqk"], c["wqn"], c["wkn"], IKc,
                                  c["pos"], top=top)
    assert not sc[0, 0, :nb].any()
    assert mask[0, 0, :top].all() and not mask[0, 0, top:nb].any()


@pytest.mark.parametrize("max_ctx,pos,top", [(16384, 12001, 512), (33024, 30001, 700), (131328, 9999, 512)])
def test_qsa_select_storage_paths(fnlib, max_ctx, pos, top):
    """The selection keeps each thread's scores in registers up to 8 blocks a thread (here 3), up to 32 (here 8, for a
    cache past 8192 blocks) and re-reads them from memory for caches past 32768 blocks."""
    _say(f"qsa select paths max_ctx={max_ctx} pos={pos} top={top}")
    c = make_case(1, 1, max_ctx, [pos], seed=5 + pos % 7)
    assert run_and_check(fnlib, c, top=top) == 1


def test_qsa_one_token_prep_inside_scoring_same_bits(fnlib):
    """One-token calls run the index query prep inside the scoring launch; a two-token call runs it as its own
    launch.  Token 0 of the two-token call sees what the one-token call sees, so its scores, its kept blocks and the
    raw key it appends must be the same bits.  Both positions complete a block (699: block 174, scored by the third
    scoring workgroup of its query; 131: block 32 by the first, which also appends the raw key) and both queries are
    sparse at top 32."""
    _say("qsa one-token prep fused vs two-token call, pos 699 / 131, top 32")
    c = make_case(2, 2, 768, [699, 131], seed=8)
    out = []
    for nt in (2, 1):
        Kc, Vc, IKc = c["Kc"].copy(), c["Vc"].copy(), c["IKc"].copy()
        og, sc, mask = fnlib.attn_qsa(c["qg"][:, :nt], c["k"][:, :nt], c["v"][:, :nt], c["wq"], c["wk"], Kc, Vc,
                                      c["iqk"][:, :nt], c["wqn"], c["wkn"], IKc, c["pos"], top=32)
        out.append((sc[:, 0], mask[:, 0], IKc))
    for b, p in enumerate((699, 131)):
        nb = (p + 1) // 4
        assert np.array_equal(out[0][0][b, :nb], out[1][0][b, :nb]), b
        assert np.array_equal(out[0][1][b], out[1][1][b]), b
        assert np.array_equal(out[0][2][b, p], out[1][2][b, p]), b
        assert np.array_equal(out[1][2][b, p], c["iqk"][b, 0, 512:]), b


def test_qsa_block_keys_written_by_one_token_calls(fnlib):
    """Consecutive one-token calls on device caches: the block keys the scoring launches write (for dense queries
    too) equal block keys rebuilt from the raw keys afterwards, bit for bit, and every call's output equals that of a
    twin whose block keys are rebuilt from its raw keys before each call.  Sequence 0 stays sparse (297 .. 302,
    completing block 74); sequence 1 starts dense at top 32 (126: 31 blocks; 127 completes block 31 while still
    dense) and turns sparse at 131, where it scores block 31 as written by the dense call and completes block 32."""
    B, nq, nkv, hd, max_ctx, top = 2, 16, 2, 256, 768, 32
    fnlib.dev_status()  # (clears bits earlier tests left)
    nsplit = fnlib.attn_nsplit(B, nkv, 1, 4 * top + 4)
    wb = fnlib.attn_qsa_work_bytes(B, nq, 1, nsplit, max_ctx, top)
    rng = np.random.default_rng(9)
    cache, ikn, bkn = B * nkv * max_ctx * hd, B * max_ctx * 128, B * max_ctx // 4 * 128
    w = {n: hiprt.Buf.like(rng.normal(1.0, 0.1, m).astype(np.float32))
         for n, m in (("wq", hd), ("wk", hd), ("wqn", 128), ("wkn", 128))}
    twins = []
    for i in range(2):
        d = {"K": hiprt.Buf.empty((cache,)), "V": hiprt.Buf.empty((cache,)), "IK": hiprt.Buf.empty((ikn,)),
             "BK": hiprt.Buf.empty((bkn,)), "work": hiprt.Buf(wb), "og": hiprt.Buf.empty((B, 1, nq, hd)),
             "pos": hiprt.Buf.empty((B,), np.int32)}
        for j, key in enumerate(("K", "V", "IK")):
            fnlib.fill_normal_dev(d[key].ptr, d[key].nbytes // 4, 40 + j)  # the same contents in both twins
        d["BK"].zero()
        fnlib.ix_blocks_dev(B, max_ctx, 0, max_ctx // 4, d["IK"].ptr, w["wkn"].ptr, d["BK"].ptr)
        twins.append(d)
    pos0 = np.array([297, 126], np.int32)
    for step in range(6):
        pos = pos0 + step
        _say(f"qsa one-token device step {step}: pos {pos.tolist()}")
        x = {n: hiprt.Buf.like(rng.standard_normal(s).astype(np.float32))
             for n, s in (("qg", (B, 1, nq, 2, hd)), ("k", (B, 1, nkv, hd)), ("v", (B, 1, nkv, hd)),
                          ("iqk", (B, 1, 640)))}
        ogs = []
        for i, d in enumerate(twins):
            if i == 1:  # the twin's block keys rebuilt from its raw keys (those not yet complete are not read)
                fnlib.ix_blocks_dev(B, max_ctx, 0, max_ctx // 4, d["IK"].ptr, w["wkn"].ptr, d["BK"].ptr)
            d["pos"].upload(pos)
            fnlib.attn_qsa_dev(B, nq, nkv, 1, max_ctx, d["pos"].ptr, x["qg"].ptr, x["k"].ptr, x["v"].ptr,
                               w["wq"].ptr, w["wk"].ptr, d["K"].ptr, d["V"].ptr, x["iqk"].ptr, w["wqn"].ptr,
                               w["wkn"].ptr, d["IK"].ptr, d["BK"].ptr, top, nsplit, d["work"].ptr, wb, d["og"].ptr)
            hiprt.sync()
            ogs.append(d["og"].download())
        assert np.array_equal(ogs[0], ogs[1]), step
        for b in x.values():
            b.free()
    assert fnlib.dev_status() == 0
    # the written block keys against a rebuild from the final raw keys, every block complete in both sequences
    a = twins[0]
    got = a["BK"].download((B, max_ctx // 4 // 64, 32, 64, 4))
    fnlib.ix_blocks_dev(B, max_ctx, 0, max_ctx // 4, a["IK"].ptr, w["wkn"].ptr, a["BK"].ptr)
    hiprt.sync()
    want = a["BK"].download((B, max_ctx // 4 // 64, 32, 64, 4))
    for b in range(B):
        nb = (int(pos0[b]) + 6) // 4
        g = got[b].transpose(0, 2, 1, 3).reshape(-1, 128)[:nb]
        r = want[b].transpose(0, 2, 1, 3).reshape(-1, 128)[:nb]
        assert np.array_equal(g, r), b
    for d in twins:
        for buf in d.values():
            buf.free()
    for buf in w.values():
        buf.free()


def test_qsa_position_outside_cache_sets_status(fnlib):
    """A new token at or past max_ctx in a sparse layer (one-token calls with the prep inside the scoring launch, and
    a three-token call): the status word records FN_STATUS_POS, that sequence's raw and block keys are left as they
    were, the other sequence appends its raw key (and, at 511, builds its last block's key), and the output is
    finite."""
    import fn

    B, nq, nkv, hd, max_ctx, top = 2, 16, 2, 256, 512, 32
    fnlib.dev_status()  # start clean
    rng = np.random.default_rng(12)
    for nt, pos in ((1, [511, 512]), (3, [505, 600])):
        _say(f"qsa position outside the cache: nt={nt} pos={pos}")
        nsplit = fnlib.attn_nsplit(B, nkv, nt, 4 * top + 4)
        wb = fnlib.attn_qsa_work_bytes(B, nq, nt, nsplit, max_ctx, top)
        cache, ikn, bkn = B * nkv * max_ctx * hd, B * max_ctx * 128, B * max_ctx // 4 * 128
        K, V = hiprt.Buf.empty((cache,)), hiprt.Buf.empty((cache,))
        IK, BK = hiprt.Buf.empty((ikn,)), hiprt.Buf.empty((bkn,))
        for j, buf in enumerate((K, V, IK, BK)):
            fnlib.fill_normal_dev(buf.ptr, buf.nbytes // 4, 60 + j)
        hiprt.sync()
        ik0, bk0 = IK.download((B, max_ctx, 128)), BK.download((B, bkn // B))
        iqk = rng.standard_normal((B, nt, 640)).astype(np.float32)
        d = {n: hiprt.Buf.like(x) for n, x in (
            ("qg", rng.standard_normal((B, nt, nq, 2, hd)).astype(np.float32)),
            ("k", rng.standard_normal((B, nt, nkv, hd)).astype(np.float32)),
            ("v", rng.standard_normal((B, nt, nkv, hd)).astype(np.float32)), ("iqk", iqk),
            ("wq", np.ones(hd, np.float32)), ("wk", np.ones(hd, np.float32)), ("wqn", np.ones(128, np.float32)),
            ("wkn", np.ones(128, np.float32)), ("pos", np.array(pos, np.int32)))}
        work, og = hiprt.Buf(wb), hiprt.Buf.empty((B, nt, nq, hd))
        fnlib.attn_qsa_dev(B, nq, nkv, nt, max_ctx, d["pos"].ptr, d["qg"].ptr, d["k"].ptr, d["v"].ptr, d["wq"].ptr,
                           d["wk"].ptr, K.ptr, V.ptr, d["iqk"].ptr, d["wqn"].ptr, d["wkn"].ptr, IK.ptr, BK.ptr, top,
                           nsplit, work.ptr, wb, og.ptr)
        assert fnlib.dev_status(clear=False) & fn.STATUS_POS
        assert fnlib.dev_status() & fn.STATUS_POS
        assert fnlib.dev_status() == 0
        assert np.isfinite(og.download()).all()
        ik, bk = IK.download((B, max_ctx, 128)), BK.download((B, bkn // B))
        assert np.array_equal(ik[1], ik0[1]) and np.array_equal(bk[1], bk0[1])  # the sequence past the cache
        p0 = pos[0]
        n_in = min(nt, max_ctx - p0)
        assert np.array_equal(ik[0, p0:p0 + n_in], iqk[0, :n_in, 512:])
        assert np.array_equal(ik[0, :p0], ik0[0, :p0])
        for x in (K, V, IK, BK, work, og, *d.values()):
            x.free()
