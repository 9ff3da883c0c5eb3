"""Device-resident decoder step / decode loop / generation against the oracle."""
import numpy as np
import pytest

from rapidocrvl_amd import lib, synth
from rapidocrvl_amd.config import ERNIE_0P3B, DecoderConfig

pytestmark = pytest.mark.gpu

Q8, Q4, Q6 = 1000, 1001, 1002
TINY = DecoderConfig(hidden=128, inter=192, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=300, eps=1e-5,
                     rope_theta=500000.0)
MID = DecoderConfig(hidden=1024, inter=3072, layers=3, heads=16, kv_heads=2, head_dim=128, vocab=5000, eps=1e-5,
                    rope_theta=500000.0)


def assert_same_choice(gt, ot, gl, ol):
    """Greedy tokens agree, unless the oracle's scores of the two picks are
    closer than twice the measured logit error (each pick's logit then moved
    by at most that error: the flip is the logit bar's, not a new one)."""
    err = float(np.max(np.abs(np.asarray(gl, np.float64) - ol)))
    assert gt == ot or float(ol[ot]) - float(ol[gt]) <= 2 * err, (gt, ot, err)


def _pair(orc, ctx, cfg, qtype, seed=3, quirk=True):
    w = synth.make_weights(cfg, qtype, seed=seed)
    om = orc.Model(cfg)
    om.load_weights(w)
    om.set_quirk(quirk)
    gm = lib.Model(ctx, cfg)
    gm.load_weights(w)
    gm.set_residual_quirk(quirk)
    return w, om, gm


def _close(got, want, rel):
    scale = max(1.0, float(np.max(np.abs(want))))
    err = float(np.max(np.abs(got - want)))
    assert err <= rel * scale, f"max err {err} (scale {scale})"


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
@pytest.mark.parametrize("cfg", [TINY, MID], ids=["tiny", "mid"])
@pytest.mark.parametrize("quirk", [True, False], ids=["quirk", "noquirk"])
def test_step_logits_and_kv(orc, ctx, cfg, qtype, quirk):
    w, om, gm = _pair(orc, ctx, cfg, qtype, quirk=quirk)
    os_, gs = om.seq(16), gm.seq(16)
    for p in range(10):  # first-token, 1..5 and >=6 branches
        emb = w["embed"][(7 * p + 3) % cfg.vocab]
        ot, ol, _ = os_.step(emb, (p, p, p))
        gt, gl = gs.step(emb, (p, p, p))
        # logits: 1e-2 max-abs and 1e-3 relative RMS (the path's stated bar)
        assert np.max(np.abs(gl - ol)) < 1e-2
        assert np.sqrt(np.mean((gl - ol) ** 2)) <= 1e-3 * np.sqrt(np.mean(ol ** 2))
        _close(gl, ol, 2e-4)
        assert gt == int(np.argmax(gl))
        assert_same_choice(gt, ot, gl, ol)
    assert len(gs) == len(os_) == 10
    for li in range(cfg.layers):
        gk, gv = gs.read_kv(li)
        ok, ov = os_.kv(li)
        assert gk.shape == ok.shape
        # row t of the cache is token t: each row matches its own token's K/V
        _close(gk.reshape(10, -1), ok.reshape(10, -1), 1e-4)
        _close(gv.reshape(10, -1), ov.reshape(10, -1), 1e-4)


@pytest.mark.parametrize("qtype", [Q4, Q6], ids=["q4", "q6"])
@pytest.mark.parametrize("quirk", [True, False], ids=["quirk", "noquirk"])
def test_step_unfused_oproj(orc, ctx, monkeypatch, qtype, quirk):
    """At the decoder's shape the step folds the attention merge into o_proj
    (per-head partial rows summed by the gate/up prologue).  The two-launch
    path (merge, then the o_proj GEMV with its residual epilogue) must meet
    the same bar against the oracle, and both paths must pick the same
    tokens."""
    w, om, gm = _pair(orc, ctx, MID, qtype, quirk=quirk)
    monkeypatch.setenv("POCR_FUSED_OPROJ", "0")
    os_, gs = om.seq(16), gm.seq(16)
    monkeypatch.delenv("POCR_FUSED_OPROJ")
    fs = gm.seq(16)
    for p in range(8):  # first-token, 1..5 and >=6 branches
        emb = w["embed"][(5 * p + 1) % MID.vocab]
        ot, ol, _ = os_.step(emb, (p, p, p))
        monkeypatch.setenv("POCR_FUSED_OPROJ", "0")
        gt, gl = gs.step(emb, (p, p, p))
        monkeypatch.delenv("POCR_FUSED_OPROJ")
        ft, fl = fs.step(emb, (p, p, p))
        for t, l in ((gt, gl), (ft, fl)):
            assert np.max(np.abs(l - ol)) < 1e-2
            assert np.sqrt(np.mean((l - ol) ** 2)) <= 1e-3 * np.sqrt(np.mean(ol ** 2))
            assert_same_choice(t, ot, l, ol)
        assert gt == ft or abs(float(fl[ft]) - float(fl[gt])) <= 2 * float(np.max(np.abs(fl - gl))), (gt, ft)


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
def test_non_final_prompt_tokens(orc, ctx, qtype):
    w, om, gm = _pair(orc, ctx, MID, qtype)
    os_, gs = om.seq(8), gm.seq(8)
    for p in range(4):
        emb = w["embed"][p + 1]
        last = p == 3
        ot, ol, _ = os_.step(emb, (p, p, p), need_logits=last)
        gt, gl = gs.step(emb, (p, p, p), need_logits=last)
    _close(gl, ol, 2e-4)
    assert gt == ot


@pytest.mark.parametrize("qtype", [Q8, Q4, Q6], ids=["q8", "q4", "q6"])
def test_generate_token_stream(orc, ctx, qtype):
    w, om, gm = _pair(orc, ctx, MID, qtype)
    ids = synth.prompt_ids(24, seed=5, high=MID.vocab)
    want = om.generate(ids, 20, eos=())
    s = gm.seq(64)
    got = s.generate(ids, 20, eos=())
    assert list(got) == list(want)
    # same stream through the device decode loop after explicit prefill steps
    s.reset()
    for p, t in enumerate(ids):
        tok, _ = s.step(w["embed"][t], (p, p, p), need_logits=p == len(ids) - 1, want_logits=False)
    got2 = s.decode_greedy(tok, len(ids), 20, eos=())
    assert list(got2) == list(want)


def test_decode_lengths_across_graph_replays(orc, ctx):
    """The greedy loop replays four token steps per graph launch and reads
    the state back every 16 steps, with single-step replays for the rest:
    every length from 1 to 40 tokens (ends inside a four-step replay, at a
    read-back, one past it) and an EOS inside a replay give the oracle's
    stream, and the cache keeps exactly the rows of the tokens before the
    stop (a second decode continues the oracle's stream)."""
    w, om, gm = _pair(orc, ctx, MID, Q4)
    ids = synth.prompt_ids(11, seed=31, high=MID.vocab)
    want = list(om.generate(ids, 40, eos=()))
    s = gm.seq(64)
    for n in (1, 2, 3, 4, 5, 7, 8, 15, 16, 17, 18, 20, 31, 33, 40):
        s.reset()
        assert list(s.generate(ids, n, eos=())) == want[:n], n
    for k in (2, 6, 13, 17):  # EOS as the (k+1)-th token: mid-replay and past a read-back
        eos = want[k]
        if eos in want[:k]:
            continue
        s.reset()
        got = list(s.generate(ids, 40, eos=(eos,)))
        assert got == want[:k + 1], k
        # the stop keeps the rows of the tokens before it: decoding on from the
        # EOS token continues the oracle's stream
        more = list(s.decode_greedy(eos, len(ids) + k, 6, eos=()))
        assert more == want[k:k + 6], k
    s.close()
    gm.close()


def test_generate_eos(orc, ctx):
    w, om, gm = _pair(orc, ctx, MID, Q4)
    ids = synth.prompt_ids(8, seed=9, high=MID.vocab)
    full = om.generate(ids, 24, eos=())
    eos = int(full[5])
    want = om.generate(ids, 24, eos=(eos,))
    s = gm.seq(64)
    got = s.generate(ids, 24, eos=(eos,))
    assert list(got) == list(want)
    assert got[-1] == eos
    # the loop stops at the EOS before any step for it (model.go:1545-1548):
    # one cache row per prompt token and per token before the EOS, although
    # the device ran its chunk of 16 steps
    assert len(s) == ids.size + len(got) - 1
    ref = gm.seq(64)
    ref.generate(ids, 24, eos=())
    for li in (0, MID.layers - 1):
        k, v = s.read_kv(li)
        rk, rv = ref.read_kv(li)
        n = k.size
        assert n == len(s) * MID.kv_rows
        assert np.array_equal(k, rk[:n]) and np.array_equal(v, rv[:n])
    # the sequence steps on from there: its next row is row len(s)
    tok, _ = s.step(w["embed"][eos], (len(s),) * 3)
    assert len(s) == ids.size + len(got)


def _eos_list(stream, cut, n_ids, vocab):
    """An EOS list of n_ids ids whose only id the stream takes is
    stream[cut], placed last (past the 16 ids the step state holds): the
    fillers are ids the stream never takes before cut, and ids at or past
    the vocabulary, which no step can take."""
    used = set(int(t) for t in stream[:cut + 1])
    fill = [t for t in range(vocab) if t not in used][: max(0, (n_ids - 1) // 2)]
    fill += list(range(vocab, vocab + (n_ids - 1 - len(fill))))
    return fill + [int(stream[cut])]


@pytest.mark.parametrize("n_ids", [1, 16, 17, 40, 1024])
def test_generate_long_eos_lists(orc, ctx, n_ids):
    """Up to maxEOSTokenIDs (1,024, model.go:432) ids; the device loop itself
    stops at the EOS (it took 6 tokens, not its chunk of 16), as with a short
    list, and the oracle stops at the same token."""
    w, om, gm = _pair(orc, ctx, MID, Q4)
    ids = synth.prompt_ids(8, seed=9, high=MID.vocab)
    full = om.generate(ids, 24, eos=())
    cut = 5
    assert int(full[cut]) not in set(int(t) for t in full[:cut])
    eos = _eos_list(full, cut, n_ids, MID.vocab)
    assert len(eos) == n_ids
    want = om.generate(ids, 24, eos=tuple(eos))
    assert list(want) == list(full[:cut + 1])
    s = gm.seq(64)
    got = s.generate(ids, 24, eos=eos)
    assert list(got) == list(want)
    assert s.device_tokens() == cut + 1
    assert len(s) == ids.size + cut
    # decode_greedy from the same state takes the same list
    s2 = gm.seq(64)
    first = int(s2.generate(ids, 1, eos=())[0])
    assert list(s2.decode_greedy(first, ids.size, 24, eos=eos)) == list(want)
    assert s2.device_tokens() == cut + 1


def test_eos_list_limits(ctx):
    """ValidateGenerateOptions (model.go:461-467): more than 1,024 ids or a
    negative id is an argument error, checked before anything runs; the
    sequence stays usable."""
    w = synth.make_weights(TINY, Q4, seed=1)
    gm = lib.Model(ctx, TINY)
    gm.load_weights(w)
    ids = synth.prompt_ids(6, seed=4, high=TINY.vocab)
    s = gm.seq(64)
    bad = [list(range(1025)), [3, -1], [-(1 << 30)]]
    for eos in bad:
        with pytest.raises(lib.PocrError) as e:
            s.generate(ids, 8, eos=eos)
        assert e.value.code == lib.POCR_ERR_ARG
        assert len(s) == 0
        with pytest.raises(lib.PocrError) as e:
            s.decode_greedy(1, 0, 5, eos=eos)
        assert e.value.code == lib.POCR_ERR_ARG
        with pytest.raises(lib.PocrError) as e:
            lib.decode_batch([s], [1], [0], 5, eos=eos)
        assert e.value.code == lib.POCR_ERR_ARG
        b = lib.Batch(gm)
        with pytest.raises(lib.PocrError) as e:
            b.join(s, 1, 0, 5, eos=eos)
        assert e.value.code == lib.POCR_ERR_ARG
        b.close()
    ok = list(s.generate(ids, 8, eos=list(range(TINY.vocab, TINY.vocab + 1024))))
    assert len(ok) == 8


def test_decode_batch_long_eos_list(ctx):
    """The batched decode stops each member on the device at the first id of
    a 40-id list it takes."""
    cfg = MID
    gm = lib.Model(ctx, cfg)
    gm.load_weights(synth.make_weights(cfg, Q4, seed=21))
    prompts = [synth.prompt_ids(n, seed=60 + n, high=cfg.vocab) for n in (17, 30, 9)]
    streams = []
    for ids in prompts:
        s = gm.seq(len(ids) + 40)
        streams.append([int(t) for t in s.generate(ids, 24, eos=(), use_prefill=True)])
        s.close()
    eos = _eos_list(streams[0], 4, 39, cfg.vocab) + [streams[1][9]]
    eset = set(eos)
    cuts = [next((i for i, t in enumerate(st) if t in eset), None) for st in streams]
    seqs = [gm.seq(len(ids) + 40) for ids in prompts]
    firsts = [int(s.generate(ids, 1, eos=(), use_prefill=True)[0]) for s, ids in zip(seqs, prompts)]
    got = [list(t) for t in lib.decode_batch(seqs, firsts, [len(i) for i in prompts], 24, eos=eos)]
    for st, cut, g, s, ids in zip(streams, cuts, got, seqs, prompts):
        if cut is None:
            assert g == st
            assert s.device_tokens() == 23
        else:
            assert g == st[:cut + 1]
            assert s.device_tokens() == cut + 1
            assert len(s) == len(ids) + cut
    assert cuts[0] is not None and cuts[0] <= 4
    for s in seqs:
        s.close()
    gm.close()


@pytest.mark.parametrize("qtype", [Q4, Q6], ids=["q4", "q6"])
def test_generate_with_image(orc, ctx, qtype):
    w, om, gm = _pair(orc, ctx, MID, qtype)
    IMG = MID.vocab - 1
    ids = np.array([5, 6, 7] + [IMG] * 12 + [8, 9, 10], np.int32)
    img = synth.image_embeds(12, MID.hidden, seed=2)
    want = om.generate(ids, 12, eos=(), image_embeds=img, image_token_id=IMG, grid=(1, 6, 8))
    got = gm.seq(64).generate(ids, 12, eos=(), image_embeds=img, image_token_id=IMG, grid=(1, 6, 8))
    assert list(got) == list(want)


def test_residual_rule_and_weights_fixed_once_sequences_exist(ctx):
    """A sequence's captured decode graphs hold the o_proj epilogue's residual
    rule and the weights' device addresses, so the model refuses to change
    either while sequences exist (setting the rule it already has is fine)
    and accepts both again once they are closed."""
    gm = lib.Model(ctx, TINY)
    gm.load_weights(synth.make_weights(TINY, Q4, seed=3))
    gm.set_residual_quirk(False)
    s = gm.seq(16)
    gm.set_residual_quirk(False)
    with pytest.raises(lib.PocrError):
        gm.set_residual_quirk(True)
    # the matrices likewise (a replaced weight could be freed under the graphs)
    with pytest.raises(lib.PocrError):
        gm.load_weights(synth.make_weights(TINY, Q4, seed=4))
    s.close()
    gm.set_residual_quirk(True)
    gm.load_weights(synth.make_weights(TINY, Q4, seed=4))
    gm.close()


def test_capacity_is_enforced(ctx):
    w = synth.make_weights(TINY, Q4, seed=1)
    gm = lib.Model(ctx, TINY)
    gm.load_weights(w)
    s = gm.seq(3)
    for p in range(3):
        s.step(w["embed"][p], (p, p, p))
    with pytest.raises(lib.PocrError) as e:
        s.step(w["embed"][0], (3, 3, 3))
    assert e.value.code == lib.POCR_ERR_ARG
    s.reset()
    with pytest.raises(lib.PocrError):
        s.decode_greedy(1, 0, 5, eos=())


def test_ernie_q8_prompt64_greedy16(orc, ctx):
    # the reference CPU workload: 18 layers, Q8, 64 ids from [0,100000) seed 0, 16 greedy tokens
    cfg = ERNIE_0P3B
    w, om, gm = _pair(orc, ctx, cfg, Q8, seed=0)
    ids = synth.prompt_ids(64, seed=0)
    orc.set_threads(8)
    want = om.generate(ids, 16, eos=())
    got = gm.seq(128).generate(ids, 16, eos=())
    assert list(got) == list(want)


def test_graph_replay_equals_direct_launches(ctx, monkeypatch):
    """The decode loop replays one captured HIP graph per token; with
    POCR_HIP_GRAPH=0 it launches the same kernels directly.  Both must give
    the same tokens and bit-identical caches, single and batched."""
    from rapidocrvl_amd import synth
    from rapidocrvl_amd.config import DecoderConfig

    cfg = DecoderConfig(hidden=1024, inter=3072, layers=3, heads=16, kv_heads=2, head_dim=128, vocab=5000,
                        eps=1e-5, rope_theta=500000.0)
    gm = lib.Model(ctx, cfg)
    gm.load_weights(synth.make_weights(cfg, lib.Q4, seed=21))
    prompts = [synth.prompt_ids(n, seed=60 + n, high=cfg.vocab) for n in (17, 30, 9, 24, 12)]

    def run():
        single = []
        for ids in prompts[:2]:
            s = gm.seq(len(ids) + 40)
            toks = list(s.generate(ids, 32, eos=(), use_prefill=True))
            single.append((toks, [s.read_kv(li) for li in (0, cfg.layers - 1)]))
            s.close()
        seqs = [gm.seq(len(ids) + 40) for ids in prompts]
        firsts = [int(s.generate(ids, 1, eos=(), use_prefill=True)[0]) for s, ids in zip(seqs, prompts)]
        batched = [list(t) for t in lib.decode_batch(seqs, firsts, [len(i) for i in prompts], 24, eos=())]
        kv = [seqs[i].read_kv(cfg.layers - 1) for i in range(len(seqs))]
        for s in seqs:
            s.close()
        return single, batched, kv

    monkeypatch.setenv("POCR_HIP_GRAPH", "1")
    g_single, g_batched, g_kv = run()
    monkeypatch.setenv("POCR_HIP_GRAPH", "0")
    d_single, d_batched, d_kv = run()
    for (gt, gkv), (dt, dkv) in zip(g_single, d_single):
        assert gt == dt
        for (gk, gv), (dk, dv) in zip(gkv, dkv):
            assert np.array_equal(gk, dk) and np.array_equal(gv, dv)
    assert g_batched == d_batched
    for (gk, gv), (dk, dv) in zip(g_kv, d_kv):
        assert np.array_equal(gk, dk) and np.array_equal(gv, dv)
    gm.close()
