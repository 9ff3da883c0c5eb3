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
