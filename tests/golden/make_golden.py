#!/usr/bin/env python3
"""Writes tests/golden/oracle_streams.json (run from the repository root:
``python tests/golden/make_golden.py``).

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


def main():
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
