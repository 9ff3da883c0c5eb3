"""Batched greedy decode (pocr_decode_batch): several sequences of one model
advance together — each layer GEMV streams its weights once for all of them,
each sequence keeps its own KV cache.  Every sequence's stream must equal the
oracle's greedy stream for that sequence alone."""
import numpy as np
import pytest

from rapidocrvl_amd import lib, synth
from rapidocrvl_amd.config import ERNIE_0P3B, DecoderConfig

pytestmark = pytest.mark.gpu

Q8, Q4, Q6 = 1000, 1001, 1002
MID = DecoderConfig(hidden=1024, inter=3072, layers=3, heads=16, kv_heads=2, head_dim=128, vocab=5000, eps=1e-5,
                    rope_theta=500000.0)
IMG = 100295


def _models(orc, ctx, cfg, qtype, seed):
    w = synth.make_weights(cfg, qtype, seed=seed)
    om = orc.Model(cfg)
    om.load_weights(w)
    gm = lib.Model(ctx, cfg)
    gm.load_weights(w)
    return om, gm


def _prefilled(gm, ids, n_new, **img):
    """A sequence after the batched prefill of ids, and its first token."""
    s = gm.seq(len(ids) + n_new + 4)
    first = s.generate(ids, 1, eos=(), use_prefill=True, **img)
    return s, int(first[0])


@pytest.mark.parametrize("qtype", [Q4, Q6, Q8], ids=["q4", "q6", "q8"])
@pytest.mark.parametrize("nseq", [2, 3, 4])
def test_decode_batch_matches_oracle(orc, ctx, qtype, nseq):
    om, gm = _models(orc, ctx, MID, qtype, seed=5)
    lens = [9, 30, 17, 41][:nseq]  # different cache lengths per sequence
    prompts = [synth.prompt_ids(n, seed=20 + i, high=MID.vocab) for i, n in enumerate(lens)]
    n_new = 20
    want = [list(om.generate(ids, n_new, eos=())) for ids in prompts]
    seqs, firsts = zip(*[_prefilled(gm, ids, n_new) for ids in prompts])
    got = lib.decode_batch(list(seqs), list(firsts), lens, n_new, eos=())
    for i in range(nseq):
        assert list(got[i]) == want[i], i
        assert len(seqs[i]) == lens[i] + n_new - 1  # one cache row per step


def test_decode_batch_eos_stops_one_sequence(orc, ctx):
    om, gm = _models(orc, ctx, MID, Q4, seed=6)
    prompts = [synth.prompt_ids(n, seed=40 + n, high=MID.vocab) for n in (12, 25)]
    full = [list(om.generate(ids, 16, eos=())) for ids in prompts]
    stop = full[0][5]  # the 6th token of sequence 0 is its EOS
    expect0 = full[0][: full[0].index(stop) + 1]
    expect1 = full[1][: full[1].index(stop) + 1] if stop in full[1] else full[1]
    seqs, firsts = zip(*[_prefilled(gm, ids, 16) for ids in prompts])
    got = lib.decode_batch(list(seqs), list(firsts), [12, 25], 16, eos=(stop,))
    assert list(got[0]) == expect0
    assert list(got[1]) == expect1
    # cache rows: the prompt's and one per token before the EOS (or the last token)
    assert len(seqs[0]) == 12 + len(expect0) - 1
    assert len(seqs[1]) == 25 + len(expect1) - 1


def test_decode_batch_rejects_bad_arguments(ctx):
    gm = lib.Model(ctx, MID)
    gm.load_weights(synth.make_weights(MID, Q4, seed=1))
    s = gm.seq(8)
    with pytest.raises(lib.PocrError):
        lib.decode_batch([s, s], [1, 2], [0, 0], 4)  # the same sequence twice
    with pytest.raises(lib.PocrError):
        lib.decode_batch([s], [MID.vocab], [0], 4)  # token outside the vocabulary
    with pytest.raises(lib.PocrError):
        lib.decode_batch([s], [1], [0], 20)  # more steps than the capacity


def test_decode_batch_ernie_images(orc, ctx):
    # the server shape in small: four image prompts (5 ids + a 4×6 merged grid
    # + 8 ids, seeds 0-3) on the full 18-layer decoder, decoded together
    cfg = ERNIE_0P3B
    om, gm = _models(orc, ctx, cfg, Q4, seed=0)
    orc.set_threads(16)
    n_new, grid = 10, (1, 8, 12)
    seqs, firsts, poss, want = [], [], [], []
    for i in range(4):
        ids = np.concatenate([synth.prompt_ids(5, seed=10 + i), np.full(24, IMG, np.int32),
                              synth.prompt_ids(8, seed=20 + i)]).astype(np.int32)
        img = synth.image_embeds(24, cfg.hidden, seed=i)
        want.append(list(om.generate(ids, n_new, eos=(), image_embeds=img, image_token_id=IMG, grid=grid)))
        s, f = _prefilled(gm, ids, n_new, image_embeds=img, image_token_id=IMG, grid=grid)
        _, delta = lib.mm_positions(ids, IMG, grid)
        seqs.append(s)
        firsts.append(f)
        poss.append(ids.size + delta)
    got = lib.decode_batch(seqs, firsts, poss, n_new, eos=())
    for i in range(4):
        assert list(got[i]) == want[i], i


# ---- continuous batching (pocr_batch_*) --------------------------------------

def _oracle_streams(om, prompts, n_new, eos=()):
    return [list(om.generate(ids, n_new, eos=eos)) for ids in prompts]


def test_continuous_batch_staggered_joins(orc, ctx):
    # members join at different token steps and with different budgets; each
    # stream equals its single-sequence greedy stream
    om, gm = _models(orc, ctx, MID, Q4, seed=7)
    lens, budgets = [11, 26, 7, 33, 19], [14, 9, 20, 6, 12]
    prompts = [synth.prompt_ids(n, seed=60 + i, high=MID.vocab) for i, n in enumerate(lens)]
    want = [list(om.generate(ids, b, eos=())) for ids, b in zip(prompts, budgets)]
    b = lib.Batch(gm)
    seqs = []
    for i in range(5):
        s, f = _prefilled(gm, prompts[i], budgets[i])
        seqs.append((s, f))
    got = {}
    b.join(seqs[0][0], seqs[0][1], lens[0], budgets[0], eos=())
    assert b.step(3) == 1
    b.join(seqs[1][0], seqs[1][1], lens[1], budgets[1], eos=())
    b.join(seqs[2][0], seqs[2][1], lens[2], budgets[2], eos=())
    assert b.step(2) == 3
    b.join(seqs[3][0], seqs[3][1], lens[3], budgets[3], eos=())
    assert b.step(1) == 4
    # the fifth member moves the batch from the 4-vector GEMV passes to the
    # wide (MFMA) step, and back once members finish
    b.join(seqs[4][0], seqs[4][1], lens[4], budgets[4], eos=())
    pending = [0, 1, 2, 3, 4]
    for _ in range(100):
        left = b.step(4)
        for i in list(pending):
            n, done = b.poll(seqs[i][0])
            assert n <= budgets[i]
            if done:
                got[i] = list(b.leave(seqs[i][0]))
                pending.remove(i)
        if not pending:
            break
        assert left >= 0
    assert sorted(got) == [0, 1, 2, 3, 4]
    for i in range(5):
        assert got[i] == want[i], i
        assert len(seqs[i][0]) == lens[i] + budgets[i] - 1
    b.close()


def test_continuous_batch_eos_and_leave_early(orc, ctx):
    om, gm = _models(orc, ctx, MID, Q6, seed=8)
    prompts = [synth.prompt_ids(n, seed=80 + n, high=MID.vocab) for n in (15, 22, 9)]
    full = _oracle_streams(om, prompts, 18)
    stop = full[0][4]
    b = lib.Batch(gm)
    seqs = [_prefilled(gm, ids, 18) for ids in prompts]
    for (s, f), ids in zip(seqs, prompts):
        b.join(s, f, ids.size, 18, eos=(stop,))
    b.step(2)
    # sequence 2 is cancelled after two steps: it has its first tokens only
    early = list(b.leave(seqs[2][0]))
    assert 1 <= len(early) <= 3 and early == full[2][:len(early)]
    while b.step(16):
        pass
    for i in (0, 1):
        exp = full[i][: full[i].index(stop) + 1] if stop in full[i] else full[i]
        n, done = b.poll(seqs[i][0])
        assert done and n == len(exp)
        assert list(b.leave(seqs[i][0])) == exp
        assert len(seqs[i][0]) == prompts[i].size + len(exp) - 1
    # a left sequence takes ordinary calls again
    seqs[2][0].reset()
    assert b.step(4) == 0
    b.close()


def test_continuous_batch_rules(ctx):
    gm = lib.Model(ctx, MID)
    gm.load_weights(synth.make_weights(MID, Q4, seed=2))
    b = lib.Batch(gm)
    s = gm.seq(16)
    ids = synth.prompt_ids(4, seed=1, high=MID.vocab)
    first = int(s.generate(ids, 1, eos=(), use_prefill=True)[0])
    with pytest.raises(lib.PocrError):  # more tokens than the capacity
        b.join(s, first, 4, 20, eos=())
    b.join(s, first, 4, 6, eos=())
    with pytest.raises(lib.PocrError):  # already a member
        b.join(s, first, 4, 6, eos=())
    with pytest.raises(lib.PocrError):  # members take no other generation call
        s.generate(ids, 2, eos=())
    with pytest.raises(lib.PocrError):
        s.reset()
    # one token is done at the join, with no device step
    t = gm.seq(16)
    first_t = int(t.generate(ids, 1, eos=(), use_prefill=True)[0])
    b.join(t, first_t, 4, 1, eos=())
    assert b.poll(t) == (1, True)
    assert list(b.leave(t)) == [first_t]
    # destroying a member removes it; the batch carries on
    b.step(1)
    s.close()
    assert b.step(4) == 0
    other = lib.Model(ctx, MID)
    other.load_weights(synth.make_weights(MID, Q4, seed=2))
    w = other.seq(16)
    with pytest.raises(lib.PocrError):  # a sequence of another model
        b.join(w, first, 4, 4, eos=())
    b.close()
    other.close()


# ---- wide batches: 5..16 sequences on the small MFMA GEMM ---------------------

@pytest.mark.parametrize("qtype,nseq", [(Q4, 5), (Q4, 8), (Q4, 16), (Q6, 16), (Q8, 11)],
                         ids=["q4-5", "q4-8", "q4-16", "q6-16", "q8-11"])
def test_decode_batch_wide_matches_oracle(orc, ctx, qtype, nseq):
    om, gm = _models(orc, ctx, MID, qtype, seed=9)
    lens = [5 + (7 * i) % 23 for i in range(nseq)]  # 5 (the Q4/Q6 in-place rows) .. 27
    prompts = [synth.prompt_ids(n, seed=100 + i, high=MID.vocab) for i, n in enumerate(lens)]
    n_new = 12
    want = [list(om.generate(ids, n_new, eos=())) for ids in prompts]
    seqs, firsts = zip(*[_prefilled(gm, ids, n_new) for ids in prompts])
    got = lib.decode_batch(list(seqs), list(firsts), lens, n_new, eos=())
    for i in range(nseq):
        assert list(got[i]) == want[i], i
        assert len(seqs[i]) == lens[i] + n_new - 1


def test_decode_batch_wide_short_prompts(orc, ctx):
    # cache lengths 1..5 keep the Q4 o_proj residual in place (model.go:3895-3902,
    # 4051-4057): each row of the wide step follows its own sequence's length
    om, gm = _models(orc, ctx, MID, Q4, seed=10)
    lens = [1, 2, 3, 4, 5, 6, 1, 3]
    prompts = [synth.prompt_ids(n, seed=200 + i, high=MID.vocab) for i, n in enumerate(lens)]
    want = [list(om.generate(ids, 10, eos=())) for ids in prompts]
    seqs, firsts = zip(*[_prefilled(gm, ids, 10) for ids in prompts])
    got = lib.decode_batch(list(seqs), list(firsts), lens, 10, eos=())
    for i in range(len(lens)):
        assert list(got[i]) == want[i], i


def test_continuous_batch_sixteen_members(orc, ctx):
    om, gm = _models(orc, ctx, MID, Q4, seed=11)
    n_req = 20
    lens = [6 + (5 * i) % 19 for i in range(n_req)]
    budgets = [4 + (3 * i) % 11 for i in range(n_req)]
    prompts = [synth.prompt_ids(n, seed=300 + i, high=MID.vocab) for i, n in enumerate(lens)]
    want = [list(om.generate(ids, bud, eos=())) for ids, bud in zip(prompts, budgets)]
    b = lib.Batch(gm)
    queue, members, got = list(range(n_req)), [], {}
    seqs = {}
    most = 0
    while queue or members:
        while queue and len(members) < 16:
            i = queue.pop(0)
            s, f = _prefilled(gm, prompts[i], budgets[i])
            seqs[i] = s
            b.join(s, f, lens[i], budgets[i], eos=())
            members.append(i)
        most = max(most, len(members))
        b.step(3)
        for i in list(members):
            if b.poll(seqs[i])[1]:
                got[i] = list(b.leave(seqs[i]))
                members.remove(i)
                seqs[i].close()
    assert most == 16
    for i in range(n_req):
        assert got[i] == want[i], i
    b.close()


def test_continuous_batch_limit(ctx):
    gm = lib.Model(ctx, MID)
    gm.load_weights(synth.make_weights(MID, Q4, seed=2))
    b = lib.Batch(gm)
    ids = synth.prompt_ids(4, seed=1, high=MID.vocab)
    seqs = []
    for i in range(17):
        s = gm.seq(16)
        first = int(s.generate(ids, 1, eos=(), use_prefill=True)[0])
        if i < 16:
            b.join(s, first, 4, 6, eos=())
        else:
            with pytest.raises(lib.PocrError):  # 16 members are decoding
                b.join(s, first, 4, 6, eos=())
        seqs.append(s)
    with pytest.raises(lib.PocrError):
        lib.decode_batch(seqs, [1] * 17, [4] * 17, 4)  # 17 sequences
    b.close()


# ---- sampling members ----------------------------------------------------------

def _sampled_prefill(gm, ids, n_new, temp, top_k, seed):
    s = gm.seq(len(ids) + n_new + 4)
    s.set_sampling(temp, top_k, seed)
    first = s.generate(ids, 1, eos=(), use_prefill=True)  # seeds the generator, draws the first token
    return s, int(first[0])


def _single_streams(om, gm, prompts, budgets, opts):
    """The streams each request may generate on its own: the oracle's stream
    for greedy ones; for sampling ones the oracle's stream or the device's
    single-sequence stream after the same batched prefill.  The batched step
    sums o_proj in another order than the single step (which folds it into
    the attention merge), so a draw within last-bit distance of a
    cumulative-weight boundary can go either way: request 1 of the mixed test
    takes the oracle's token at draw 12, the single device path its
    neighbour.  The single sampled path is checked against the oracle in
    test_gpu_sampling.py."""
    out = []
    for ids, bud, (t, k, sd) in zip(prompts, budgets, opts):
        if t > 0:
            s = gm.seq(len(ids) + bud + 4)
            s.set_sampling(t, k, sd)
            dev = list(s.generate(ids, bud, eos=(), use_prefill=True))
            s.close()
            out.append([dev, list(om.generate(ids, bud, eos=(), temperature=t, top_k=k, seed=sd))])
        else:
            out.append([list(om.generate(ids, bud, eos=()))])
    return out


@pytest.mark.parametrize("nseq", [3, 8], ids=["narrow", "wide"])
def test_decode_batch_mixes_greedy_and_sampling(orc, ctx, nseq):
    # every other sequence draws from its top-k (its own generator, continued
    # from its prefill's draw); each stream equals its single-sequence stream
    om, gm = _models(orc, ctx, MID, Q4, seed=12)
    lens = [7 + 3 * i for i in range(nseq)]
    prompts = [synth.prompt_ids(n, seed=400 + i, high=MID.vocab) for i, n in enumerate(lens)]
    opts = [(0.0, 0, 0) if i % 2 == 0 else (0.7 + 0.1 * i, 8 + 4 * i, 1000 + i) for i in range(nseq)]
    n_new = 14
    want = _single_streams(om, gm, prompts, [n_new] * nseq, opts)
    seqs, firsts = [], []
    for ids, (t, k, sd) in zip(prompts, opts):
        s, f = _sampled_prefill(gm, ids, n_new, t, k, sd) if t > 0 else _prefilled(gm, ids, n_new)
        seqs.append(s)
        firsts.append(f)
    got = lib.decode_batch(seqs, firsts, lens, n_new, eos=())
    for i in range(nseq):
        assert list(got[i]) in want[i], (i, opts[i])


def test_continuous_batch_sampling_members(orc, ctx):
    om, gm = _models(orc, ctx, MID, Q6, seed=13)
    n_req = 7
    lens = [9 + 2 * i for i in range(n_req)]
    budgets = [6 + 2 * i for i in range(n_req)]
    prompts = [synth.prompt_ids(n, seed=500 + i, high=MID.vocab) for i, n in enumerate(lens)]
    opts = [(0.9, 16, 77 + i) if i % 3 else (0.0, 0, 0) for i in range(n_req)]
    want = _single_streams(om, gm, prompts, budgets, opts)
    b = lib.Batch(gm)
    queue, members, got, seqs = list(range(n_req)), [], {}, {}
    while queue or members:
        while queue and len(members) < 5:
            i = queue.pop(0)
            t, k, sd = opts[i]
            s, f = (_sampled_prefill(gm, prompts[i], budgets[i], t, k, sd) if t > 0
                    else _prefilled(gm, prompts[i], budgets[i]))
            seqs[i] = s
            b.join(s, f, lens[i], budgets[i], eos=())
            members.append(i)
        b.step(4)
        for i in list(members):
            if b.poll(seqs[i])[1]:
                got[i] = list(b.leave(seqs[i]))
                members.remove(i)
    for i in range(n_req):
        assert got[i] in want[i], (i, opts[i])
    b.close()


# a vocabulary in 16-row blocks: more than 4 greedy rows take the MFMA LM head
# (logits rows + per-row argmax) instead of the 4-vector GEMV passes
MID16 = DecoderConfig(hidden=1024, inter=3072, layers=3, heads=16, kv_heads=2, head_dim=128, vocab=5008, eps=1e-5,
                      rope_theta=500000.0)


@pytest.mark.parametrize("qtype,nseq", [(Q4, 6), (Q4, 16), (Q8, 9)], ids=["q4-6", "q4-16", "q8-9"])
def test_decode_batch_mfma_lm_head(orc, ctx, qtype, nseq):
    om, gm = _models(orc, ctx, MID16, qtype, seed=14)
    lens = [3 + (11 * i) % 29 for i in range(nseq)]
    prompts = [synth.prompt_ids(n, seed=600 + i, high=MID16.vocab) for i, n in enumerate(lens)]
    want = [list(om.generate(ids, 12, eos=())) for ids in prompts]
    seqs, firsts = zip(*[_prefilled(gm, ids, 12) for ids in prompts])
    got = lib.decode_batch(list(seqs), list(firsts), lens, 12, eos=())
    for i in range(nseq):
        assert list(got[i]) == want[i], i


def test_decode_batch_mfma_lm_head_with_sampling(orc, ctx):
    # 12 sequences, 8 greedy (MFMA head) and 4 sampling (their own heads)
    om, gm = _models(orc, ctx, MID16, Q4, seed=15)
    nseq = 12
    lens = [5 + 2 * i for i in range(nseq)]
    prompts = [synth.prompt_ids(n, seed=700 + i, high=MID16.vocab) for i, n in enumerate(lens)]
    opts = [(0.85, 10, 50 + i) if i % 3 == 1 else (0.0, 0, 0) for i in range(nseq)]
    want = _single_streams(om, gm, prompts, [10] * nseq, opts)
    seqs, firsts = [], []
    for ids, (t, k, sd) in zip(prompts, opts):
        s, f = _sampled_prefill(gm, ids, 10, t, k, sd) if t > 0 else _prefilled(gm, ids, 10)
        seqs.append(s)
        firsts.append(f)
    got = lib.decode_batch(seqs, firsts, lens, 10, eos=())
    for i in range(nseq):
        assert list(got[i]) in want[i], (i, opts[i])


def test_decode_batch_long_and_wide_sampling_members(orc, ctx):
    # six sequences (the wide MFMA step), 128 tokens each: greedy members
    # beside members drawing from every logit (top_k 0, top_k >= vocab), from
    # 300 sorted candidates and from 20; each stream equals its
    # single-sequence stream
    om, gm = _models(orc, ctx, MID, Q4, seed=16)
    opts = [(0.0, 0, 0), (0.8, 0, 31), (1.0, 300, 32), (0.0, 0, 0), (1.1, MID.vocab, 33), (0.9, 20, 34)]
    nseq = len(opts)
    lens = [6 + 5 * i for i in range(nseq)]
    prompts = [synth.prompt_ids(n, seed=800 + i, high=MID.vocab) for i, n in enumerate(lens)]
    n_new = 128
    want = _single_streams(om, gm, prompts, [n_new] * nseq, opts)
    seqs, firsts = [], []
    for ids, (t, k, sd) in zip(prompts, opts):
        s, f = _sampled_prefill(gm, ids, n_new, t, k, sd) if t > 0 else _prefilled(gm, ids, n_new)
        seqs.append(s)
        firsts.append(f)
    got = lib.decode_batch(seqs, firsts, lens, n_new, eos=())
    for i in range(nseq):
        assert list(got[i]) in want[i], (i, opts[i])
    for s in seqs:
        s.close()
