"""One model driven from several host threads at once.

The reference's server runs requests for one loaded model from several
goroutines (internal/model/model.go's Generate on per-request state); here
every entry point takes the context's lock, each thread owns its sequences,
and the weights are shared.  Each thread's tokens must equal what the same
calls give when run one after another on one thread."""
import threading

import numpy as np
import pytest

from rapidocrvl_amd import lib, synth
from rapidocrvl_amd.config import DecoderConfig

pytestmark = pytest.mark.gpu

Q4 = 1001
MID = DecoderConfig(hidden=1024, inter=3072, layers=3, heads=16, kv_heads=2, head_dim=128, vocab=5000, eps=1e-5,
                    rope_theta=500000.0)
LENS = [7, 19, 33, 12, 26, 40]
# greedy, top-40, every logit, a wide candidate set
SETTINGS = [(0.0, 0, 0), (0.8, 40, 11), (0.0, 0, 0), (1.0, 0, 12), (0.7, 200, 13), (0.0, 0, 0)]


def _request(gm, i, ids):
    """Prefill + 24 tokens, then the per-token path for 10 more from scratch."""
    s = gm.seq(len(ids) + 32)
    s.set_sampling(*SETTINGS[i])
    a = list(s.generate(ids, 24, eos=(), use_prefill=True))
    s.close()
    s = gm.seq(len(ids) + 16)
    s.set_sampling(*SETTINGS[i])
    b = list(s.generate(ids, 10, eos=(), use_prefill=False))
    s.close()
    return a, b


def _batch(gm, prompts):
    """Three greedy sequences through one batched decode."""
    seqs = [gm.seq(len(ids) + 24) for ids in prompts]
    firsts = [int(s.generate(ids, 1, eos=(), use_prefill=True)[0]) for s, ids in zip(seqs, prompts)]
    got = lib.decode_batch(seqs, firsts, [len(ids) for ids in prompts], 16, eos=())
    for s in seqs:
        s.close()
    return [list(g) for g in got]


def _ops(ctx, rng_seed):
    """Op-level calls on the shared context: top-k draws over fixed logits."""
    rng = np.random.default_rng(rng_seed)
    logits = rng.standard_normal(5000).astype(np.float32)
    out, state = [], 99
    for _ in range(20):
        tok, state = ctx.sample_topk(logits, 40, 0.8, state)[:2]
        out.append(int(tok))
    return out


def test_threads_share_one_model(ctx):
    w = synth.make_weights(MID, Q4, seed=8)
    gm = lib.Model(ctx, MID)
    gm.load_weights(w)
    prompts = [synth.prompt_ids(n, seed=70 + i, high=MID.vocab) for i, n in enumerate(LENS)]
    batch_prompts = [synth.prompt_ids(n, seed=90 + n, high=MID.vocab) for n in (11, 23, 5)]
    jobs = [(lambda i=i: _request(gm, i, prompts[i])) for i in range(len(LENS))]
    jobs.append(lambda: _batch(gm, batch_prompts))
    jobs.append(lambda: _ops(ctx, 5))
    serial = [job() for job in jobs]

    rounds = 2
    results = [[None] * len(jobs) for _ in range(rounds)]
    errors = []
    start = threading.Barrier(len(jobs))

    def worker(j):
        try:
            start.wait()
            for r in range(rounds):
                results[r][j] = jobs[j]()
        except BaseException as e:  # reported below with the job's index
            errors.append((j, repr(e)))

    threads = [threading.Thread(target=worker, args=(j,)) for j in range(len(jobs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=300)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    for r in range(rounds):
        for j in range(len(jobs)):
            assert results[r][j] == serial[j], (r, j)
    gm.close()
