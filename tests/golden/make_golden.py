#!/usr/bin/env python3
"""Writes tests/golden/oracle_streams.json (run from the repository root:
``python tests/golden/make_golden.py``) and, with ``--full``,
tests/golden/oracle_streams_full.json: the greedy streams of the two
image-conditioned workloads at their real sizes (about 15 minutes on 8 cores).

The reference is pure Go and cannot run here, and its tests hold no golden
token streams, so these streams come from the oracle (the C restatement of the
reference's CPU decoder, itself pinned by reference_kats.json and the float64
decoder in tests/decoder_f64.py).  They give the GPU path fixed targets and pin
the oracle against silent changes.  Every input is seeded synthetic data:
weights from rapidocrvl_amd.synth.make_weights (N(0,0.02) f32 → bf16 → row
quantized with the half-away encoder), prompt ids from synth.prompt_ids.

reference_kats.json is not generated: it restates known answers from the
reference's own tests, each with its source file and line.
"""
import dataclasses
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from rapidocrvl_amd import synth  # noqa: E402
from rapidocrvl_amd.config import ERNIE_0P3B, DecoderConfig  # noqa: E402

Q8, Q4, Q6 = 1000, 1001, 1002
QN = {Q8: "q8", Q4: "q4", Q6: "q6"}
TINY = DecoderConfig(hidden=128, inter=192, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=300, eps=1e-5,
                     rope_theta=500000.0)
TINY_IMAGE_TOKEN = 299


def tiny_cases():
    """(name, cfg, qtype, weight seed, quirk, ids, image rows, grid, max_new)"""
    ids = synth.prompt_ids(12, seed=3, high=TINY.vocab - 1)
    out = [(f"tiny_{QN[q]}", TINY, q, 3, True, ids, None, None, 8) for q in (Q8, Q6, Q4)]
    out.append(("tiny_q4_noquirk", TINY, Q4, 3, False, ids, None, None, 8))
    img_ids = np.array([5, 6] + [TINY_IMAGE_TOKEN] * 4 + [7, 8], np.int32)
    out.append(("tiny_q4_image", TINY, Q4, 3, True, img_ids, synth.image_embeds(4, TINY.hidden, seed=0),
                (1, 4, 4), 6))
    return out


def ernie_cases():
    ids = synth.prompt_ids(64, seed=0)
    return [(f"ernie_{QN[q]}_prompt64", ERNIE_0P3B, q, 0, True, ids, None, None, 16) for q in (Q8, Q4)]


def run_case(case, weights):
    name, cfg, qtype, seed, quirk, ids, img, grid, max_new = case
    m = oracle.Model(cfg)
    m.load_weights(weights)
    m.set_quirk(quirk)
    kw = {}
    if img is not None:
        kw = dict(image_embeds=img, image_token_id=TINY_IMAGE_TOKEN, grid=grid)
    toks = m.generate(ids, max_new, eos=(), **kw)
    rec = {"config": dataclasses.asdict(cfg), "qtype": qtype, "weight_seed": seed,
           "quirk": quirk, "ids": [int(i) for i in ids], "max_new": max_new, "tokens": [int(t) for t in toks]}
    if img is not None:
        rec.update(image_rows=int(img.shape[0]), image_seed=0, image_token_id=TINY_IMAGE_TOKEN, grid=list(grid))
    if cfg is TINY and img is None:
        # logits of the last prompt token (one step per prompt token)
        s = m.seq(len(ids) + 1)
        for p, t in enumerate(ids):
            last = p == len(ids) - 1
            _, logits, _ = s.step(weights["embed"][t], (p, p, p), need_logits=last)
        rec["last_prompt_logits"] = [float(v) for v in logits]
    m.close()
    return name, rec


IMAGE_TOKEN = 100295
IMAGE_GRID = (1, 72, 74)  # 36 x 37 merged patches = 1332 visual rows


def image_prompt(head_seed, n_head, tail_seed, n_tail):
    """n_head ids, 1332 image placeholders, n_tail ids (ids uniform in [0, 100000))."""
    return np.concatenate([synth.prompt_ids(n_head, seed=head_seed), np.full(1332, IMAGE_TOKEN, np.int32),
                           synth.prompt_ids(n_tail, seed=tail_seed)]).astype(np.int32)


def full_cases():
    """(name, qtype, ids, image seed, max_new, (head seed, n_head, tail seed, n_tail)).

    image_q4_1345: 5 ids + 1332 visual rows + 8 ids, one 1345-token prefill and
    256 greedy tokens (the batch-1 decode workload).  serve_{q4,q6}_{i}: four
    server-style requests, 5 ids (seed 100+i) + 1332 visual rows (seed i) +
    11 ids (seed 200+i), 1024 greedy tokens each, caches growing to 2372 rows."""
    out = [("image_q4_1345", Q4, image_prompt(0, 5, 1, 8), 0, 256, (0, 5, 1, 8))]
    for qtype in (Q4, Q6):
        for i in range(4):
            out.append((f"serve_{QN[qtype]}_{i}", qtype, image_prompt(100 + i, 5, 200 + i, 11), i, 1024,
                        (100 + i, 5, 200 + i, 11)))
    # a request whose greedy choice at token 315 is a near tie (top-2 logits
    # 4.8e-5 apart): 5 ids (seed 314) + 1332 visual rows (seed 314) + 11 ids
    # (seed 414), through token 315
    out.append(("near_tie_q4_314", Q4, image_prompt(314, 5, 414, 11), 314, 316, (314, 5, 414, 11)))
    return out


def stream_with_gaps(m, weights, ids, img, max_new):
    """The oracle's greedy generation (generate_impl's loop: one step per
    prompt token, then one per new token at position len(out)-1+ropeDelta),
    keeping each chosen token's top-2 logit gap."""
    pos, delta = oracle.mm_positions(ids, IMAGE_TOKEN, IMAGE_GRID)
    s = m.seq(len(ids) + max_new)
    j = 0
    for p, t in enumerate(ids):
        if t == IMAGE_TOKEN:
            emb = img[j]
            j += 1
        else:
            emb = weights["embed"][t]
        last = p == len(ids) - 1
        tok, lg, _ = s.step(emb, pos[p], need_logits=last, want_logits=last)
    assert j == img.shape[0]
    toks, gaps = [], []
    while True:
        top2 = np.partition(lg, -2)[-2:]
        assert int(np.argmax(lg)) == tok
        toks.append(int(tok))
        gaps.append(float(top2.max() - top2.min()))
        if len(toks) == max_new:
            break
        p = len(ids) + len(toks) - 1 + delta
        tok, lg, _ = s.step(weights["embed"][tok], (p, p, p))
    return toks, gaps, len(ids) + delta


def main_full():
    from rapidocrvl_amd.config import ERNIE_0P3B as cfg

    oracle.set_threads(min(16, os.cpu_count() or 1))
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle_streams_full.json")
    cases = {}
    if os.path.exists(path) and "--redo" not in sys.argv[1:]:  # keep the cases already written
        with open(path) as f:
            cases = json.load(f)["cases"]
    weights = {}
    for name, qtype, ids, img_seed, max_new, prompt in full_cases():
        if name in cases:
            continue
        if qtype not in weights:
            weights = {qtype: synth.make_weights(cfg, qtype, seed=0)}
            m = oracle.Model(cfg)
            m.load_weights(weights[qtype])
        img = synth.image_embeds(1332, cfg.hidden, seed=img_seed)
        toks, gaps, first_pos = stream_with_gaps(m, weights[qtype], ids, img, max_new)
        if name == "image_q4_1345":  # the step loop is the oracle's own generation loop
            assert list(m.generate(ids, 4, eos=(), image_embeds=img, image_token_id=IMAGE_TOKEN,
                                   grid=IMAGE_GRID)) == toks[:4]
        near = [[k, g] for k, g in enumerate(gaps) if g < 1e-3]
        cases[name] = {"qtype": qtype, "weight_seed": 0, "prompt": {"head_seed": prompt[0], "n_head": prompt[1],
                                                                     "tail_seed": prompt[2], "n_tail": prompt[3]},
                       "image_rows": 1332, "image_seed": img_seed, "image_token_id": IMAGE_TOKEN,
                       "grid": list(IMAGE_GRID), "prompt_len": int(ids.size), "first_pos": int(first_pos),
                       "max_new": max_new, "tokens": toks, "min_top2_gap": min(gaps),
                       "near_ties": near}
        print(name, "min gap %.3g" % min(gaps), "near", near, toks[:12], flush=True)
        write_full(path, cfg, cases)


def write_full(path, cfg, cases):
    out = {"_about": "Greedy streams of the oracle for the ERNIE 0.3B decoder (seeded synthetic weights) on "
                     "image-conditioned prompts at full size, with each token's top-2 logit gap below 1e-3; "
                     "written by make_golden.py --full.",
           "config": dataclasses.asdict(cfg), "cases": cases}
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", path, flush=True)


def main():
    if "--full" in sys.argv[1:]:
        main_full()
        return
    oracle.set_threads(min(16, os.cpu_count() or 1))
    cases = {}
    cache = {}
    for case in tiny_cases() + ernie_cases():
        key = (id(case[1]), case[2], case[3])
        if key not in cache:
            cache[key] = synth.make_weights(case[1], case[2], seed=case[3])
        name, rec = run_case(case, cache[key])
        cases[name] = rec
        print(name, rec["tokens"], flush=True)
    out = {"_about": "Greedy streams of the oracle for seeded synthetic models; written by make_golden.py.",
           "cases": cases}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle_streams.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
