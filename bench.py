#!/usr/bin/env python3
"""Batch-1 greedy decode throughput of the 0.3B ERNIE text decoder (Q4) on one
MI355X, plus the quantized-GEMV roofline and the CPU baseline.

Workload (the image-conditioned OCR generation): 5 text ids, 1332 visual-token
embeddings (N(0,1), a 36×37 merged grid from a 72×74 patch grid), 8 text ids
→ one 1345-token prefill, then greedy decode of 256 tokens at batch 1 with the
KV cache growing 1345 → 1600.  One timed step = one 256-token decode from the
same prefilled state; EOS is disabled so every step emits 256 tokens.
Weights are seeded synthetic N(0,0.02) bf16, row-quantized to Q4 (and Q8 for
the secondary figure).

Roofline kernel: the greedy Q4 LM-head GEMV (103424×1024, M=1, argmax — the
launch the decode loop runs), timed with HIP events on the library stream while
rotating through copies whose total exceeds the 256 MB Infinity Cache.  CPU baseline: the oracle (a C restatement of the
reference's pure-Go CPU path) decoding from the same prefilled KV state on the
host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
IMAGE_TOKEN = 100295


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def workload_ids():
    from rapidocrvl_amd import synth

    head = synth.prompt_ids(5, seed=0)
    tail = synth.prompt_ids(8, seed=1)
    return np.concatenate([head, np.full(1332, IMAGE_TOKEN, np.int32), tail]).astype(np.int32)


def batch_decode(model, cfg, n_seq=4, n_new=1024, reps=2):
    """Server-style generation: n_seq independent sequences (5 ids + 1332 visual
    rows + 11 ids, seeds 0..n_seq-1), each prefilled, then greedy-decoded
    together for n_new tokens (one device step per token for all of them: the
    layer GEMVs run at M = n_seq).  Returns aggregate tok/s of the last rep."""
    from rapidocrvl_amd import lib, synth

    grid = (1, 72, 74)
    seqs, firsts, poss, n_pre = [], [], [], []
    for i in range(n_seq):
        ids = np.concatenate([synth.prompt_ids(5, seed=100 + i), np.full(1332, IMAGE_TOKEN, np.int32),
                              synth.prompt_ids(11, seed=200 + i)]).astype(np.int32)
        img = synth.image_embeds(1332, cfg.hidden, seed=i)
        s = model.seq(ids.size + n_new + 8)
        first = s.generate(ids, 1, eos=(), image_embeds=img, image_token_id=IMAGE_TOKEN, grid=grid,
                           use_prefill=True)
        _, delta = lib.mm_positions(ids, IMAGE_TOKEN, grid)
        seqs.append(s)
        firsts.append(int(first[0]))
        poss.append(ids.size + delta)
        n_pre.append(ids.size)
    dt = None
    for _ in range(reps):
        for s, n in zip(seqs, n_pre):
            s.truncate(n)
        t = time.perf_counter()
        out = lib.decode_batch(seqs, firsts, poss, n_new, eos=())
        dt = time.perf_counter() - t
        assert all(len(o) == n_new for o in out)
    # every member's first tokens against the same request decoded alone
    # (pocr_decode_greedy, one sequence per step), after the timed runs
    n_check = min(n_new, 256)
    splits = []
    for i, (s, n) in enumerate(zip(seqs, n_pre)):
        s.truncate(n)
        alone = s.decode_greedy(firsts[i], poss[i], n_check, eos=())
        diff = np.nonzero(np.asarray(alone[:n_check]) != np.asarray(out[i][:n_check]))[0]
        if diff.size:
            splits.append({"sequence": i, "index": int(diff[0])})
    for s in seqs:
        s.close()
    return {"sequences": n_seq, "tokens_each": n_new, "context": f"{n_pre[0]}->{n_pre[0] + n_new}",
            "tok_s": round(n_seq * n_new / dt, 1), "ms_per_step": round(dt / (n_new - 1) * 1e3, 4),
            "tokens_match_alone": not splits, "checked_tokens_each": n_check, "splits": splits}


SERVE_BUDGETS = (512, 128, 384, 256, 640, 192, 448, 320)


_EMBED = {}


def model_embed(model, tok):
    """Embedding row of a token of the bench's synthetic Q4 model (seed 0)."""
    from rapidocrvl_amd import synth

    key = id(model)
    if key not in _EMBED:
        _EMBED.clear()
        _EMBED[key] = synth.normal((model.cfg.vocab, model.cfg.hidden), [0, 1000, 2])
    return _EMBED[key][tok]


def serve(model, cfg, budgets=SERVE_BUDGETS, slots=4, chunk=16, seed0=300, sample_every=0, eos=()):
    """Server-style serving of len(budgets) image requests (5 ids + 1332 visual
    rows + 11 ids, seeds 300+i; request i generates budgets[i] greedy tokens):
    one request at a time (prefill, then its own decode loop: the reference
    server with one run slot) against continuous batching (requests prefilled
    as slots free up, joining and leaving a 4-member decode batch between
    token steps).  Wall time covers prefills and decodes; tokens/s counts
    generated tokens.  Each request's tokens must be the same both ways.
    With eos, a request stops at its first EOS token (the device turns the
    rest of the step block into no-ops) and tokens/s counts what was emitted."""
    from rapidocrvl_amd import lib, synth

    grid = (1, 72, 74)
    reqs = []
    for i, n in enumerate(budgets):
        ids = np.concatenate([synth.prompt_ids(5, seed=seed0 + i), np.full(1332, IMAGE_TOKEN, np.int32),
                              synth.prompt_ids(11, seed=seed0 + 100 + i)]).astype(np.int32)
        _, delta = lib.mm_positions(ids, IMAGE_TOKEN, grid)
        reqs.append((ids, synth.image_embeds(1332, cfg.hidden, seed=seed0 + i), ids.size + delta, n))
    seqs = [model.seq(ids.size + n + 8) for ids, _, _, n in reqs]
    # with sample_every = k, request i with i % k == 1 draws from its top 40 at T 0.8
    samples = [bool(sample_every) and i % sample_every == 1 for i in range(len(reqs))]

    def first_token(s, ids, img, i):
        s.reset()
        s.set_sampling(*((0.8, 40, 1000 + i) if samples[i] else (0.0, 0, 0)))
        return int(s.generate(ids, 1, eos=(), image_embeds=img, image_token_id=IMAGE_TOKEN, grid=grid,
                              use_prefill=True)[0])

    if eos == "auto":  # the token request 0 emits at index 100 (or its last)
        ids, img, pos, n = reqs[0]
        s0 = list(seqs[0].decode_greedy(first_token(seqs[0], ids, img, 0), pos, n, eos=()))
        eos = (int(s0[min(100, len(s0) - 1)]),)
    t = time.perf_counter()
    one = []
    for i, (s, (ids, img, pos, n)) in enumerate(zip(seqs, reqs)):
        one.append(list(s.decode_greedy(first_token(s, ids, img, i), pos, n, eos=eos)))
    t_one = time.perf_counter() - t

    t = time.perf_counter()
    b = lib.Batch(model)
    queue, members, got = list(range(len(reqs))), [], {}
    while queue or members:
        while queue and len(members) < slots:
            i = queue.pop(0)
            ids, img, pos, n = reqs[i]
            b.join(seqs[i], first_token(seqs[i], ids, img, i), pos, n, eos=eos)
            members.append(i)
        b.step(chunk)
        for i in list(members):
            if b.poll(seqs[i])[1]:
                got[i] = list(b.leave(seqs[i]))
                members.remove(i)
    t_cb = time.perf_counter() - t
    b.close()
    # a request whose two streams differ: the single-sequence logits at the
    # first differing token, top-2 gap (greedy choice between near-equal logits)
    differ = []
    for i in range(len(reqs)):
        if got[i] == one[i]:
            continue
        k = next(j for j in range(len(one[i])) if j >= len(got[i]) or got[i][j] != one[i][j])
        ids, img, pos, n = reqs[i]
        s = seqs[i]
        if samples[i]:  # a draw: near-tied neighbours or a pick close to a boundary
            differ.append({"request": i, "token": k, "of": n, "sampled": True, "single": int(one[i][k]),
                           "batched": int(got[i][k]) if k < len(got[i]) else None,
                           **draw_margin(model, s, first_token(s, ids, img, i), pos, k, 1000 + i,
                                         int(got[i][k]) if k < len(got[i]) else None)})
            continue
        toks = list(s.decode_greedy(first_token(s, ids, img, i), pos, k, eos=())) if k > 0 else []
        gap = None
        if k > 0:
            _, lg = s.step(model_embed(model, toks[k - 1]), (pos + k - 1,) * 3)
            t2 = np.sort(lg)[-2:]
            gap = float(t2[1] - t2[0])
        differ.append({"request": i, "token": k, "of": n, "single_top2_gap": gap,
                       "single_top2_rel_gap": None if gap is None else gap / max(abs(float(t2[1])), 1e-30)})
    for s in seqs:
        s.close()
    total = sum(len(o) for o in one)
    return {"requests": len(budgets), "tokens": total, "budget_tokens": sum(budgets), "eos": list(eos),
            "stopped_at_eos": sum(len(o) < n for o, (_, _, _, n) in zip(one, reqs)),
            "slots": slots, "sampling_requests": sum(samples),
            "one_at_a_time": {"s": round(t_one, 3), "tok_s": round(total / t_one, 1)},
            "continuous_batch": {"s": round(t_cb, 3), "tok_s": round(total / t_cb, 1)},
            "speedup": round(t_one / t_cb, 2),
            "tokens_match": not differ,
            "greedy_tokens_match": not any(not d.get("sampled") for d in differ), "differ": differ}


def splitmix_u(seed, k):
    """fastRNG's k-th Float64 draw from seed (model.go:1829-1840)."""
    m = (1 << 64) - 1
    z = (seed + (k + 1) * 0x9E3779B97F4A7C15) & m
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    z ^= z >> 31
    return (z >> 11) / float(1 << 53)


def draw_margin(model, s, first, pos, k, seed, batched=None, top_k=40, temperature=0.8):
    """Where the single-sequence path's draw k fell: its logits row (the prefix
    replayed), the draw u (fastRNG at the request's seed; draw 0 was the
    prefill's), the rank whose cumulative interval holds u·Σw, and the distance
    of u·Σw to the nearest cumulative boundary as a fraction of Σw (f64
    weights: a diagnostic, not the reference's f32/f64 order).  The candidates
    are ordered by score, so two tokens whose scores differ by less than the
    batched/single logit difference (a few 1e-5 here) can trade ranks: the
    same u then names the other token however far it is from a boundary.
    ``tie_gap`` is |score(single) − score(batched)| with ``adjacent`` telling
    whether the two sit at neighbouring ranks; a split with a large gap and a
    large margin would point at the batched path itself."""
    if k == 0:
        return {"margin": None}
    toks = list(s.decode_greedy(first, pos, k, eos=()))
    _, lg = s.step(model_embed(model, toks[k - 1]), (pos + k - 1,) * 3)
    order = np.lexsort((np.arange(lg.size), -lg))[:top_k]
    sc = lg[order].astype(np.float64)
    w = np.exp((sc - sc[0]) / temperature)
    cum = np.cumsum(w)
    pick = splitmix_u(seed, k) * cum[-1]
    rank = min(int(np.searchsorted(cum, pick)), top_k - 1)
    out = {"margin": float(np.min(np.abs(cum - pick)) / cum[-1]), "draw": k, "rank": rank,
           "pick_of_single_logits": int(order[rank])}
    if batched is not None:
        rb = np.flatnonzero(order == batched)
        out["tie_gap"] = float(abs(float(lg[batched]) - float(lg[order[rank]])))
        out["adjacent"] = bool(rb.size and abs(int(rb[0]) - rank) == 1)
    return out


def build_model(ctx, cfg, qtype, seed=0):
    from rapidocrvl_amd import lib, synth

    t = time.time()
    w = synth.make_weights(cfg, qtype, seed=seed)
    m = lib.Model(ctx, cfg)
    m.load_weights(w)
    log(f"[bench] weights q{ {1000: 8, 1001: 4, 1002: 6}[qtype]} ready in {time.time() - t:.1f}s")
    return w, m


PREFILL_FLOPS_PER_TOKEN_LAYER = 2 * 14_155_776  # q,k,v,o,gate,up,down weights of one layer


def projector_bench(ctx, with_cpu=True):
    """The vision projector (mlp_AR) at PaddleOCR-VL's widths (vision 1152 →
    4608 → 1024) on the bench image grid (1, 72, 74) → 1332 rows: device time
    per image, useful TFLOP/s (2·rows·(4608² + 1024·4608)), and the oracle's
    single-thread rows/s on a 6-row sample."""
    from rapidocrvl_amd import lib

    import oracle

    vd, td, grid = 1152, 1024, (1, 72, 74)
    K = 4 * vd
    rng = np.random.default_rng(11)
    w1 = (rng.standard_normal((K, K)) * (1.5 / np.sqrt(K))).astype(np.float32)
    w2 = (rng.standard_normal((td, K)) * (1.0 / np.sqrt(K))).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(vd)).astype(np.float32)
    nb = (0.1 * rng.standard_normal(vd)).astype(np.float32)
    b1 = (0.1 * rng.standard_normal(K)).astype(np.float32)
    b2 = (0.1 * rng.standard_normal(td)).astype(np.float32)
    proj = lib.Projector(ctx, nw, nb, w1, b1, w2, b2)
    us = proj.time_project(grid, iters=20)
    rows = grid[0] * (grid[1] // 2) * (grid[2] // 2)
    flops = 2.0 * rows * (K * K + td * K)
    res = {"workload": "vision projector, 1332 rows (grid 1x72x74), 1152->4608->1024, Q8",
           "ms": round(us / 1e3, 3), "TFLOP_s": round(flops / (us * 1e-6) / 1e12, 1)}
    if with_cpu:
        sample = (1, 2, 12)  # 6 rows
        x = rng.standard_normal((12 * 2, vd)).astype(np.float32)
        q1 = lib.quantize_rows(lib.Q8, w1)
        q2 = lib.quantize_rows(lib.Q8, w2)
        t = time.perf_counter()
        oracle.project_image(x, sample, nw, nb, q1, b1, q2, b2)
        dt = time.perf_counter() - t
        res["cpu_oracle_rows_s"] = round(6 / dt, 1)
        res["cpu_oracle_threads"] = 1
    proj.close()
    return res


def prefill_flops(cfg, n):
    """Linear layers 2·N·weights, causal attention 2·(QKᵀ + PV) = 4·dim·N(N+1)/2
    per head and layer, LM head on the last token."""
    lin = PREFILL_FLOPS_PER_TOKEN_LAYER * n * cfg.layers
    attn = 2 * cfg.head_dim * n * (n + 1) * cfg.heads * cfg.layers
    return lin + attn + 2 * cfg.vocab * cfg.hidden


def prefill(seq, ids, img, reps=1):
    """Batched prefill of the prompt (+ its first greedy token); the last of
    `reps` runs is timed (the first allocates the prefill buffers)."""
    for _ in range(reps):
        seq.reset()
        t = time.perf_counter()
        tok = seq.generate(ids, 1, eos=(), image_embeds=img, image_token_id=IMAGE_TOKEN, grid=(1, 72, 74),
                           use_prefill=True)
        dt = time.perf_counter() - t
    return int(tok[0]), dt


def time_decode(seq, n_prefix, first_tok, first_pos, n_tokens, warmup, steps):
    toks = None
    for _ in range(warmup):
        seq.truncate(n_prefix)
        toks = seq.decode_greedy(first_tok, first_pos, n_tokens, eos=())
    t = time.perf_counter()
    for _ in range(steps):
        seq.truncate(n_prefix)
        toks = seq.decode_greedy(first_tok, first_pos, n_tokens, eos=())
    dt = time.perf_counter() - t
    assert len(toks) == n_tokens
    return dt, toks


def gemv_rotation(ctx, q, target_bytes=600 << 20, iters=None, m=1):
    """Average µs of one GEMV launch (M rows of x) rotating over copies of q."""
    wbytes = q.packed.nbytes + q.scales.nbytes
    n = max(2, int(np.ceil(target_bytes / wbytes)))
    copies = [ctx.upload(q) for _ in range(n)]
    x = np.random.default_rng(0).standard_normal((m, q.cols)).astype(np.float32)
    iters = iters or max(4 * n, 200)
    us = ctx.time_matvec(copies, x[0], iters) if m == 1 else ctx.time_matvec_batched(copies, x, iters)
    for c in copies:
        c.close()
    return us, wbytes


def gemv_sweep(ctx, rng):
    """The four decoder GEMV shapes × Q8/Q6/Q4 × M ∈ {1, 4, 16} (M > 1: digit
    planes + MFMA GEMM); GB/s of algorithmic bytes (weights + scales + M·(x + y))."""
    from rapidocrvl_amd import lib

    shapes = {"gate_up": (3072, 1024), "down": (1024, 3072), "qkv": (2560, 1024), "lm_head": (103424, 1024)}
    out = {}
    for qname, qtype in (("q8", lib.Q8), ("q6", lib.Q6), ("q4", lib.Q4)):
        for sname, (rows, cols) in shapes.items():
            w = (rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02))
            q = lib.QMatrix.quantize(w, qtype)
            for m in (1, 4, 16):
                us, wbytes = gemv_rotation(ctx, q, m=m)
                alg = wbytes + 4 * m * (rows + cols)
                out[f"{qname}_{sname}_m{m}"] = {"us": round(us, 3), "GB/s": round(alg / us / 1e3, 1),
                                                "TOP/s": round(2 * m * rows * cols / us / 1e6, 2)}
    return out


def attention_sweep(ctx, cfg):
    """Decode attention (RoPE, K/V append, GQA over L fp32 rows) at
    L ∈ {1024, 4096, 8192}, rotating over the model's 18 layer caches."""
    out = {}
    for L in (1024, 4096, 8192):
        us = ctx.time_attention(cfg.heads, cfg.kv_heads, cfg.head_dim, L, cfg.layers, 400)
        alg = 2 * L * cfg.kv_heads * cfg.head_dim * 4 + 4 * (cfg.heads + 2 * cfg.kv_heads) * cfg.head_dim
        out[f"L{L}"] = {"us": round(us, 3), "GB/s": round(alg / us / 1e3, 1)}
    return out


def lm_head_q4(cfg, seed=0, qtype=None):
    """The Q4 (or qtype) LM head of the synthetic 0.3B weights (same draw as make_weights)."""
    from rapidocrvl_amd import lib, synth

    qt = lib.Q4 if qtype is None else qtype
    lm = synth.normal((cfg.vocab, cfg.hidden), [seed, 1000, 0])
    s, p = lib.quantize_rows(qt, lm)
    return lib.QMatrix(qt, cfg.vocab, cfg.hidden, s, p)


def q6_head(ctx, cfg):
    """The Q6 greedy LM head (the 4-sequence Q6 decode's head at M = 1), timed as
    the Q4 roofline kernel is, with the lean read of the same bytes beside it."""
    from rapidocrvl_amd import lib

    lmq = lm_head_q4(cfg, qtype=lib.Q6)
    us, alg, achieved = lm_head_roofline(ctx, lmq)
    stream_us = stream_read_ceiling(ctx, int(alg))
    return {"kernel": "k_head_mfma: q6 lm_head greedy head 103424x1024 m=1 (rows from the head image)",
            "us_per_launch": round(us, 3), "algorithmic_bytes": int(alg), "achieved_GB_s": round(achieved, 1),
            "frac": round(achieved / HBM_PEAK_GBS, 4), "stream_read_us": round(stream_us, 3),
            "frac_of_stream_read": round(stream_us / us, 4)}


def lm_head_roofline(ctx, lmq, target_bytes=600 << 20):
    """The greedy LM-head launch the decode loop runs (argmax, no logits
    written), rotating over copies whose total exceeds the Infinity Cache.
    Algorithmic bytes: weights + row scales + x."""
    wbytes = lmq.packed.nbytes + lmq.scales.nbytes
    n = max(2, int(np.ceil(target_bytes / wbytes)))
    copies = [ctx.upload(lmq) for _ in range(n)]
    x = np.random.default_rng(0).standard_normal(lmq.cols).astype(np.float32)
    trials = sorted(ctx.time_matvec_argmax(copies, x, max(4 * n, 200)) for _ in range(5))
    us = trials[len(trials) // 2]  # median of 5 timed batches
    for c in copies:
        c.close()
    alg = wbytes + 4 * lmq.cols
    return us, alg, alg / us / 1e3


def stream_read_ceiling(ctx, nbytes, target_bytes=600 << 20):
    """A plain 16-byte streaming read of nbytes (rounded up to 16) timed the
    same way as the GEMV (rotating buffers past the Infinity Cache, median of
    5 batches): the ceiling a single launch of that size reaches on this chip."""
    nbytes = (nbytes + 15) // 16 * 16
    n = max(2, int(np.ceil(target_bytes / nbytes)))
    trials = sorted(ctx.time_stream_read(nbytes, n, max(4 * n, 200)) for _ in range(5))
    return trials[len(trials) // 2]


def measured_traffic():
    """HBM bytes per launch of the roofline kernel, from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE passes (scaled by the copy-kernel factor)."""
    path = os.path.join(ROOT, "profiles", "lm_head_q4_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


def copy_calibration(nbytes=512 << 20, reps=3):
    """A plain device copy of known size (read nbytes, write nbytes): the
    reference point that scales the FETCH_SIZE/WRITE_SIZE counters.  HIP's own
    device-to-device copy (the runtime's blit kernel) is used through ctypes."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so")
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    for ptr in (src, dst):
        if hip.hipMalloc(ctypes.byref(ptr), ctypes.c_size_t(nbytes)) != 0:
            raise RuntimeError("hipMalloc failed")
    try:
        if hip.hipMemset(src, 1, ctypes.c_size_t(nbytes)) != 0:
            raise RuntimeError("hipMemset failed")
        for _ in range(reps):
            if hip.hipMemcpy(dst, src, ctypes.c_size_t(nbytes), 3) != 0:  # hipMemcpyDeviceToDevice
                raise RuntimeError("hipMemcpy failed")
        hip.hipDeviceSynchronize()
    finally:
        hip.hipFree(src)
        hip.hipFree(dst)
    log(f"[bench] copy calibration: {reps} device copies of {nbytes} bytes")


def roofline_only(args):
    """Only the roofline kernel: the Q4 LM-head GEMV rotation (the command the
    committed rocprofv3 summaries profile)."""
    from rapidocrvl_amd import lib
    from rapidocrvl_amd.config import ERNIE_0P3B as cfg

    ctx = lib.Context(0)
    lmq = lm_head_q4(cfg)
    us, alg, achieved = lm_head_roofline(ctx, lmq)
    log(f"[bench] q4 lm_head gemv {us:.2f} us → {achieved:.0f} GB/s")
    stream_us = stream_read_ceiling(ctx, int(alg))
    if args.calibrate_copy:
        copy_calibration()
    print(json.dumps({"kernel": "k_head_mfma: q4 lm_head greedy head 103424x1024 m=1", "us_per_launch": round(us, 3),
                      "algorithmic_bytes": int(alg), "achieved_GB_s": round(achieved, 1),
                      "frac": round(achieved / HBM_PEAK_GBS, 4), "stream_read_us": round(stream_us, 3),
                      "frac_of_stream_read": round(stream_us / us, 4)}), flush=True)


def vnni_decode(ctx, cfg, weights, seq, first_tok, first_pos, n_prefix, n_tokens, steps, prompt=None):
    """The same Q4 greedy decode in the reference's VNNI activation mode
    (pocr_model_set_vnni: u8 activations for every Q4 matvec, the
    reference's VNNI matvec arithmetic, with the portable scalar orders
    around it), from the same
    1345-row KV state, on its own copy of the weights.  With prompt = (ids,
    image rows), the same prompt's prefill in that mode is timed too (the
    mode's batched prefill, bit-identical to its token steps)."""
    from rapidocrvl_amd import lib

    m = lib.Model(ctx, cfg)
    m.load_weights(weights)
    m.set_vnni(True)
    extra = {}
    if prompt is not None:
        sp = m.seq(n_prefix + 8)
        tok, t_pf = prefill(sp, prompt[0], prompt[1], reps=3)
        sp.close()
        extra = {"prefill_ms": round(t_pf * 1e3, 3), "prefill_first_token": tok}
    s = m.seq(n_prefix + n_tokens + 8)
    rows = n_prefix * cfg.kv_heads * cfg.head_dim
    for li in range(cfg.layers):
        k, v = seq.read_kv(li)
        s.write_kv(li, k[:rows], v[:rows], n_prefix)
    dt, toks = time_decode(s, n_prefix, first_tok, first_pos, n_tokens, 1, steps)
    s.close()
    m.close()
    computed = n_tokens - 1
    return {"value": round(computed * steps / dt, 1), "unit": "tok/s",
            "us_per_token": round(dt / steps / computed * 1e6, 1), **extra}, [int(t) for t in toks]


def cpu_baseline(cfg, weights, gpu_seq, first_tok, first_pos, gpu_tokens, n_prefix, budget_s=12.0,
                 gpu_vnni_tokens=None):
    import oracle

    threads = min(16, os.cpu_count() or 1)
    oracle.set_threads(threads)
    t0 = time.time()
    om = oracle.Model(cfg)
    om.load_weights(weights)
    kv = [gpu_seq.read_kv(li) for li in range(cfg.layers)]
    log(f"[bench] oracle ready in {time.time() - t0:.1f}s ({threads} threads)")

    def run(n_max):
        s = om.seq(n_prefix + 64)
        for li, (k, v) in enumerate(kv):
            s.load(li, k[: n_prefix * cfg.kv_rows], v[: n_prefix * cfg.kv_rows], n_prefix)
        toks = [first_tok]
        t = time.perf_counter()
        n = 0
        while n < 4 or (time.perf_counter() - t < budget_s / 2 and n < n_max):
            p = first_pos + n
            tok, _, _ = s.step(weights["embed"][toks[-1]], (p, p, p), want_logits=False)
            toks.append(tok)
            n += 1
        return n, time.perf_counter() - t, toks

    n, dt, toks = run(48)
    match = toks[: n + 1] == list(gpu_tokens[: n + 1])
    # the same steps in the reference's u8-activation mode for Q4/Q6 matrices
    # (quantizeXForVNNI + VPDPBUSD dots, quant.go:2087-2115), which the Go
    # binary runs on an AVX512-VNNI host
    om.set_vnni(True)
    nv, dtv, toksv = run(n)
    om.set_vnni(False)
    return {"value": round(n / dt, 2), "unit": "tok/s", "cores": threads, "kind": "port",
            "host": f"{host_cpu()}, {os.cpu_count()} logical CPUs visible; {threads} worker threads "
                    f"(the GOMAXPROCS-equivalent of the pool)",
            "sample": f"{n} greedy Q4 decode steps of the 18-layer decoder from the same 1345-token KV state "
                      f"(oracle, C restatement of the pure-Go CPU path, {threads} threads)",
            "tokens_match_gpu": bool(match),
            "vnni_emulation": {"value": round(nv / dtv, 2), "unit": "tok/s", "steps": nv,
                               "tokens_match_gpu_vnni_mode": (None if gpu_vnni_tokens is None else
                                                              toksv[: nv + 1] == list(gpu_vnni_tokens[: nv + 1]))}}


GEMV_SHAPES = {"gate_up": (3072, 1024), "down": (1024, 3072), "qkv": (2560, 1024), "lm_head": (103424, 1024)}


def cpu_gemv_sweep(rng, budget_s=0.2):
    """The GEMV sweep on the CPU: the oracle's matvec (plain-mode MatVecQ*,
    quant.go:443-561) at the sweep's shapes × Q8/Q6/Q4, one vector per call
    (M rows cost M calls on the CPU path); µs per call and GB/s of weight
    bytes, each cell timed for about budget_s."""
    import oracle
    from rapidocrvl_amd import lib

    threads = min(16, os.cpu_count() or 1)
    oracle.set_threads(threads)
    cells = {}
    for qname, qtype in (("q8", lib.Q8), ("q6", lib.Q6), ("q4", lib.Q4)):
        for sname, (rows, cols) in GEMV_SHAPES.items():
            w = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
            q = lib.QMatrix.quantize(w, qtype)
            x = rng.standard_normal(cols).astype(np.float32)
            pm = oracle.Prepared(qtype, q.scales, q.packed, cols)  # unpacked once, as the model holds it
            y = np.zeros(rows, np.float32)
            pm.matvec(x, y)
            n, t = 0, time.perf_counter()
            while n < 2 or time.perf_counter() - t < budget_s:
                pm.matvec(x, y)
                n += 1
            us = (time.perf_counter() - t) / n * 1e6
            pm.close()
            cells[f"{qname}_{sname}_m1"] = {"us": round(us, 1),
                                            "GB/s": round((q.packed.nbytes + q.scales.nbytes) / us / 1e3, 2)}
    return {"threads": threads, "kind": "port", "cells": cells,
            "note": "M = 4 and 16 cost 4 and 16 calls of the m1 cell on the CPU path"}


def cpu_attention_sweep(cfg, rng, budget_s=0.3):
    """Decode attention on the CPU at L = 1k/4k/8k: the oracle's cache
    attention (model.go:4623-5590: 16 q heads over 2 kv heads, head_dim 128,
    FastExp softmax) over N(0,1) K/V, one layer per call."""
    import oracle

    threads = min(16, os.cpu_count() or 1)
    oracle.set_threads(threads)
    kvd = cfg.kv_heads * cfg.head_dim
    out = {}
    for L in (1024, 4096, 8192):
        k = rng.standard_normal(L * kvd).astype(np.float32)
        v = rng.standard_normal(L * kvd).astype(np.float32)
        q = rng.standard_normal(cfg.heads * cfg.head_dim).astype(np.float32)
        n, t = 0, time.perf_counter()
        while n < 2 or time.perf_counter() - t < budget_s:
            oracle.cache_attention(q, k, v, L, cfg.heads, cfg.kv_heads, cfg.head_dim)
            n += 1
        us = (time.perf_counter() - t) / n * 1e6
        out[f"L{L}"] = {"us": round(us, 1), "GB/s": round(2 * L * kvd * 4 / us / 1e3, 2)}
    return {"threads": threads, "kind": "port", "per_layer": out}


def cpu_worker_main(args):
    """One CPU decode worker of cpu_concurrent_workers (a child process: no
    GPU use).  Loads the Q4 weights and the KV state the parent saved, waits
    for the start file, decodes greedily for args.worker_seconds, prints one
    JSON line."""
    import oracle
    from rapidocrvl_amd import synth
    from rapidocrvl_amd.config import ERNIE_0P3B as cfg

    d = args.cpu_worker
    oracle.set_threads(args.worker_threads)
    st = np.load(os.path.join(d, "state.npz"))
    n_prefix, first_tok, first_pos = (int(v) for v in st["meta"])
    weights = synth.make_weights(cfg, synth.lib.Q4, seed=0)
    om = oracle.Model(cfg)
    om.load_weights(weights)
    s = om.seq(n_prefix + 1100)
    for li in range(cfg.layers):
        s.load(li, st[f"k{li}"], st[f"v{li}"], n_prefix)
    open(os.path.join(d, f"ready{args.worker_id}"), "w").close()
    while not os.path.exists(os.path.join(d, "go")):
        time.sleep(0.01)
    toks, n, t = [first_tok], 0, time.perf_counter()
    while n < 1024 and (n < 2 or time.perf_counter() - t < args.worker_seconds):
        p = first_pos + n
        tok, _, _ = s.step(weights["embed"][toks[-1]], (p, p, p), want_logits=False)
        toks.append(tok)
        n += 1
    dt = time.perf_counter() - t
    print(json.dumps({"worker": args.worker_id, "steps": n, "s": dt, "tokens": toks[:9]}), flush=True)


def cpu_concurrent_workers(cfg, gpu_seq, first_tok, first_pos, n_prefix, gpu_tokens, workers=4, seconds=8.0):
    """Four single-sequence CPU decode workers at once, as the reference
    server runs one GenerateWithOptions per acquired slot
    (cmd/paddleocrvl-server/main.go:1106-1124): four child processes of the
    oracle sharing the host's cores (each with cores/4 threads), each decoding
    from the same 1,345-row Q4 KV state the GPU produced.  Aggregate tok/s over
    the common decode window (the workers start together once all are
    loaded)."""
    import subprocess
    import tempfile

    threads = max(1, min(16, os.cpu_count() or 1) // workers)
    with tempfile.TemporaryDirectory(dir="/tmp") as d:
        arrs = {"meta": np.array([n_prefix, first_tok, first_pos], np.int64)}
        for li in range(cfg.layers):
            k, v = gpu_seq.read_kv(li)
            arrs[f"k{li}"] = k[: n_prefix * cfg.kv_rows]
            arrs[f"v{li}"] = v[: n_prefix * cfg.kv_rows]
        np.savez(os.path.join(d, "state.npz"), **arrs)
        env = dict(os.environ, OMP_NUM_THREADS=str(threads))
        procs = [subprocess.Popen([sys.executable, os.path.abspath(__file__), "--cpu-worker", d,
                                   "--worker-id", str(i), "--worker-threads", str(threads),
                                   "--worker-seconds", str(seconds)],
                                  stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, env=env)
                 for i in range(workers)]
        t0 = time.time()
        while not all(os.path.exists(os.path.join(d, f"ready{i}")) for i in range(workers)):
            if any(p.poll() is not None for p in procs) or time.time() - t0 > 300:
                for p in procs:
                    p.kill()
                raise RuntimeError("a CPU worker did not get ready: "
                                   + " | ".join((p.stderr.read() or "")[-300:] for p in procs if p.poll() is not None))
            time.sleep(0.05)
        open(os.path.join(d, "go"), "w").close()
        outs = []
        for p in procs:
            o, e = p.communicate(timeout=seconds + 120)
            if p.returncode != 0:
                raise RuntimeError(f"CPU worker failed: {e[-500:]}")
            outs.append(json.loads(o.strip().splitlines()[-1]))
    steps = sum(o["steps"] for o in outs)
    window = max(o["s"] for o in outs)
    match = all(o["tokens"] == list(gpu_tokens[: len(o["tokens"])]) for o in outs)
    return {"value": round(steps / window, 2), "unit": "tok/s", "cores": threads * workers, "kind": "port",
            "workers": workers, "threads_per_worker": threads,
            "per_worker_tok_s": [round(o["steps"] / o["s"], 2) for o in outs],
            "sample": f"{workers} oracle processes, each {threads} threads, decoding greedily for ≈{seconds:.0f} s "
                      f"from the same 1345-token Q4 KV state",
            "tokens_match_gpu": bool(match)}


def host_cpu():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_config1(cfg, weights_q8, gpu_model):
    """The reference's own CPU workload: Q8, 64 ids from [0,100000) seed 0,
    greedy 16 tokens — timed on the oracle, tokens compared with the GPU's.
    (The reference's u8-activation VNNI mode applies to Q4/Q6 matrices only,
    so Q8 has a single mode; the Q4 decode baseline times both.)"""
    import oracle
    from rapidocrvl_amd import synth

    threads = min(16, os.cpu_count() or 1)
    oracle.set_threads(threads)
    ids = synth.prompt_ids(64, seed=0)
    gpu = list(gpu_model.seq(96).generate(ids, 16, eos=(), use_prefill=True))
    out = {"workload": "q8, 64 prompt ids (seed 0), 16 greedy tokens, 18 layers", "threads": threads}
    for mode in ("plain",):
        om = oracle.Model(cfg)
        om.load_weights(weights_q8)
        t = time.perf_counter()
        toks = list(om.generate(ids, 16, eos=()))
        dt = time.perf_counter() - t
        out[mode] = {"s": round(dt, 3), "tok_s_end_to_end": round(16 / dt, 2),
                     "tokens_match_gpu": toks == gpu}
        om.close()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--decode-tokens", type=int, default=256)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-q8", action="store_true")
    ap.add_argument("--roofline-only", action="store_true", help="time only the Q4 LM-head GEMV rotation")
    ap.add_argument("--calibrate-copy", action="store_true", help="with --roofline-only: add a 512 MiB copy")
    ap.add_argument("--q6-head-only", action="store_true", help="time only the Q6 greedy LM head and its lean read")
    ap.add_argument("--prefill-only", action="store_true", help="time only the 1345-token Q4 image prefill")
    ap.add_argument("--decode-only", action="store_true",
                    help="time only the prefill and the Q4 greedy decode (the kernel sequence the profiles trace)")
    ap.add_argument("--no-batch", action="store_true", help="skip the 4-sequence batched decode")
    ap.add_argument("--batch-only", action="store_true", help="time only the 4-sequence Q4 batched decode")
    ap.add_argument("--projector-only", action="store_true", help="time only the vision projector")
    ap.add_argument("--attention-only", action="store_true",
                    help="time only the decode attention + merge at 1k/4k/8k cache rows")
    ap.add_argument("--serve-only", action="store_true", help="time only the 8-request serving comparison")
    ap.add_argument("--vnni-only", action="store_true",
                    help="time only the Q4 decode in the VNNI activation mode (after the plain-mode prefill)")
    ap.add_argument("--batch-tokens", type=int, default=1024, help="tokens per sequence of the batched decode")
    ap.add_argument("--batch-seqs", default="4,8,16", help="with --batch-only: batch sizes to time")
    ap.add_argument("--cpu-worker", help=argparse.SUPPRESS)  # one process of cpu_concurrent_workers
    ap.add_argument("--worker-id", type=int, default=0, help=argparse.SUPPRESS)
    ap.add_argument("--worker-threads", type=int, default=4, help=argparse.SUPPRESS)
    ap.add_argument("--worker-seconds", type=float, default=8.0, help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.cpu_worker:  # a child of cpu_concurrent_workers: CPU only
        cpu_worker_main(args)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the decoder step runs on a single MI355X "
              "(multi-GPU sharding is a design note, not built)", file=sys.stderr)
        sys.exit(2)
    if args.roofline_only:
        roofline_only(args)
        return
    if args.q6_head_only:
        from rapidocrvl_amd import lib
        from rapidocrvl_amd.config import ERNIE_0P3B as cfg

        print(json.dumps(q6_head(lib.Context(0), cfg)), flush=True)
        return

    from rapidocrvl_amd import lib, synth
    from rapidocrvl_amd.config import ERNIE_0P3B as cfg

    ctx = lib.Context(0)
    if args.projector_only:
        print(json.dumps(projector_bench(ctx, with_cpu=not args.no_cpu)), flush=True)
        return
    if args.attention_only:
        print(json.dumps({"workload": "decode attention (RoPE, K/V append, split attention + merge), 16q/2kv "
                                      "heads, 18 layer caches rotated", **attention_sweep(ctx, cfg)}), flush=True)
        return
    if args.batch_only:
        _, model = build_model(ctx, cfg, lib.Q4)
        for n in (int(v) for v in args.batch_seqs.split(",")):
            print(json.dumps({"workload": f"{n}-sequence q4 batched greedy decode",
                              **batch_decode(model, cfg, n_seq=n, n_new=args.batch_tokens, reps=1)}), flush=True)
        return
    if args.serve_only:
        _, model = build_model(ctx, cfg, lib.Q4)
        print(json.dumps({"workload": "q4 serving of 8 image requests", **serve(model, cfg)}), flush=True)
        print(json.dumps({"workload": "q4 serving of 24 image requests, 16 slots",
                          **serve(model, cfg, budgets=SERVE_BUDGETS * 3, slots=16)}), flush=True)
        print(json.dumps({"workload": "q4 serving of 24 image requests, 16 slots, every third sampling",
                          **serve(model, cfg, budgets=SERVE_BUDGETS * 3, slots=16, sample_every=3)}), flush=True)
        return
    ids = workload_ids()
    img = synth.image_embeds(1332, cfg.hidden, seed=0)
    pos, delta = lib.mm_positions(ids, IMAGE_TOKEN, (1, 72, 74))
    n_prefix = ids.size
    first_pos = n_prefix + delta

    weights, model = build_model(ctx, cfg, lib.Q4)
    seq = model.seq(n_prefix + args.decode_tokens + 8)
    first_tok, t_prefill = prefill(seq, ids, img, reps=3)
    log(f"[bench] prefill {n_prefix} tokens in {t_prefill * 1e3:.1f} ms, first token {first_tok}")
    if args.prefill_only:
        print(json.dumps({"workload": f"q4 image prefill, {n_prefix} tokens", "prefill_ms": round(t_prefill * 1e3, 3),
                          "prefill_tok_s": round(n_prefix / t_prefill, 1),
                          "prefill_TFLOP_s": round(prefill_flops(cfg, n_prefix) / t_prefill / 1e12, 2),
                          "first_token": first_tok}), flush=True)
        return
    if args.vnni_only:
        vd, _ = vnni_decode(ctx, cfg, weights, seq, first_tok, first_pos, n_prefix, args.decode_tokens,
                            max(1, args.steps // 2), prompt=(ids, img))
        print(json.dumps({"workload": f"q4 greedy decode in the VNNI activation mode, {args.decode_tokens - 1} token "
                                      f"steps after a {n_prefix}-token prefill", **vd}), flush=True)
        return
    dt, toks = time_decode(seq, n_prefix, first_tok, first_pos, args.decode_tokens, args.warmup, args.steps)
    # a step returns decode_tokens tokens, the first of them the prefill's: it
    # computes decode_tokens − 1 token steps
    computed = args.decode_tokens - 1
    tok_s = computed * args.steps / dt
    log(f"[bench] q4 decode {tok_s:.1f} tok/s ({dt / args.steps * 1e3:.1f} ms per {computed} token steps)")
    if args.decode_only:
        print(json.dumps({"workload": f"q4 greedy decode, {computed} token steps after a {n_prefix}-token prefill",
                          "tok_s": round(tok_s, 1), "us_per_token": round(dt / args.steps / computed * 1e6, 2),
                          "prefill_ms": round(t_prefill * 1e3, 3)}), flush=True)
        return
    # the reference bench's figure: generated tokens over the request's wall
    # time, prefill included (cmd/paddleocrvl-bench/main.go:499-505)
    e2e_tok_s = args.decode_tokens / (t_prefill + dt / args.steps)
    # the same decode drawing every token from the top 40 candidates (T = 0.8),
    # and from every logit (top_k 0, the reference CLI's default)
    sampled = {}
    for k in (40, 0):
        seq.set_sampling(0.8, k, 1)
        dts, _ = time_decode(seq, n_prefix, first_tok, first_pos, args.decode_tokens, 1, max(1, args.steps // 2))
        sampled[k] = computed * max(1, args.steps // 2) / dts
        log(f"[bench] q4 sampled decode (top_k {k}, T 0.8) {sampled[k]:.1f} tok/s")
    seq.set_sampling(0.0, 0, 0)

    # roofline: Q4 LM-head GEMV, rotating copies > Infinity Cache
    lm_qt, lm_sc, lm_data, lm_cols = weights["lm_head"]
    lmq = lib.QMatrix(lm_qt, lm_sc.size, lm_cols, lm_sc, lm_data)
    us, alg, achieved = lm_head_roofline(ctx, lmq)
    log(f"[bench] q4 lm_head gemv {us:.2f} us → {achieved:.0f} GB/s")
    stream_us = stream_read_ceiling(ctx, int(alg))
    log(f"[bench] plain streaming read of the same {alg} bytes: {stream_us:.2f} us")

    extra = {}
    extra["vnni_decode"], vnni_toks = vnni_decode(ctx, cfg, weights, seq, first_tok, first_pos, n_prefix,
                                                  args.decode_tokens, max(1, args.steps // 2), prompt=(ids, img))
    log(f"[bench] q4 decode in the VNNI activation mode {extra['vnni_decode']}")
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(cfg, weights, seq, first_tok, first_pos, toks, n_prefix, gpu_vnni_tokens=vnni_toks)
        log(f"[bench] cpu baseline {cpu}")
        # the other configurations' CPU legs: GEMV sweep, decode attention,
        # four concurrent single-sequence workers
        cpu["per_config"] = {"gemv_sweep": cpu_gemv_sweep(np.random.default_rng(0)),
                             "attention": cpu_attention_sweep(cfg, np.random.default_rng(1)),
                             "concurrent_workers_q4": cpu_concurrent_workers(cfg, seq, first_tok, first_pos,
                                                                             n_prefix, toks)}
        log(f"[bench] cpu per-config baselines {cpu['per_config']}")

    if not args.no_batch:
        extra["batch4_decode"] = {"q4": batch_decode(model, cfg, n_new=args.batch_tokens)}
        log(f"[bench] 4-sequence batched decode q4 {extra['batch4_decode']['q4']}")
        extra["batch_wide_decode"] = {str(n): batch_decode(model, cfg, n_seq=n, n_new=512) for n in (8, 16)}
        log(f"[bench] 8/16-sequence batched decode q4 {extra['batch_wide_decode']}")
        extra["serving_q4"] = serve(model, cfg)
        log(f"[bench] serving q4 {extra['serving_q4']}")
        extra["serving_q4_16slots"] = serve(model, cfg, budgets=SERVE_BUDGETS * 3, slots=16)
        log(f"[bench] serving q4, 16 slots {extra['serving_q4_16slots']}")
        extra["serving_q4_16slots_sampling"] = serve(model, cfg, budgets=SERVE_BUDGETS * 3, slots=16, sample_every=3)
        log(f"[bench] serving q4, 16 slots, every third request sampling {extra['serving_q4_16slots_sampling']}")
        # EOS on: the token request 0 emits at index 100 ends every request
        # whose stream reaches it
        extra["serving_q4_16slots_eos"] = serve(model, cfg, budgets=SERVE_BUDGETS * 3, slots=16, eos="auto")
        log(f"[bench] serving q4, 16 slots, EOS {extra['serving_q4_16slots_eos']}")
        _, m6 = build_model(ctx, cfg, lib.Q6)
        extra["batch4_decode"]["q6"] = batch_decode(m6, cfg, n_new=args.batch_tokens)
        log(f"[bench] 4-sequence batched decode q6 {extra['batch4_decode']['q6']}")
        m6.close()
        del m6
    if not args.no_q8:
        model.close()
        seq.close()
        w8, m8 = build_model(ctx, cfg, lib.Q8)
        s8 = m8.seq(n_prefix + args.decode_tokens + 8)
        t8, _ = prefill(s8, ids, img)
        dt8, _ = time_decode(s8, n_prefix, t8, first_pos, args.decode_tokens, 1, max(1, args.steps // 2))
        extra["q8_decode_tok_s"] = round(computed * max(1, args.steps // 2) / dt8, 1)
        s8.close()
        if not args.no_cpu:
            extra["cpu_config1"] = cpu_config1(cfg, w8, m8)
            log(f"[bench] cpu config 1 {extra['cpu_config1']}")
        m8.close()
        del w8
    extra["sampled_decode_tok_s"] = {"temperature": 0.8, "top_k_40": round(sampled[40], 1),
                                     "top_k_0_full_vocabulary": round(sampled[0], 1)}
    extra["end_to_end_tok_s"] = {"value": round(e2e_tok_s, 1), "tokens": args.decode_tokens,
                                 "s": round(t_prefill + dt / args.steps, 4),
                                 "note": "generated tokens / (prefill + decode wall time), the reference bench's tps"}
    extra["prefill_ms"] = round(t_prefill * 1e3, 2)
    extra["prefill_tok_s"] = round(n_prefix / t_prefill, 1)
    extra["prefill_TFLOP_s"] = round(prefill_flops(cfg, n_prefix) / t_prefill / 1e12, 2)

    extra["projector"] = projector_bench(ctx, with_cpu=not args.no_cpu)
    log(f"[bench] projector {extra['projector']}")
    if not args.no_sweep:
        extra["gemv_sweep"] = gemv_sweep(ctx, np.random.default_rng(0))
        extra["attention_sweep"] = attention_sweep(ctx, cfg)
        extra["q6_lm_head"] = q6_head(ctx, cfg)
        log(f"[bench] q6 lm_head {extra['q6_lm_head']}")

    per_token_bytes = 181_542_912 + 36_864 * (n_prefix + args.decode_tokens // 2)
    result = {
        "metric": "decode tok/s at batch 1 (Q4/Q8) + quant-GEMV achieved HBM GB/s vs peak",
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 3),
        "tokens_per_step": computed,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4 weight codes x int8 activation digit planes (3 planes, int32 dot, f32 scale/accumulate)",
        "data": "synthetic",
        "config": {"workload": "ernie-0.3b q4 greedy decode, batch 1, 256 tokens after a 1345-token "
                               "image+text prefill (5 ids + 1332 visual rows + 8 ids)",
                   "layers": cfg.layers, "hidden": cfg.hidden, "heads": f"{cfg.heads}q/{cfg.kv_heads}kv",
                   "context": f"{n_prefix}->{n_prefix + args.decode_tokens}", "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel": "k_head_mfma: q4 lm_head greedy head (int8 MFMA over 3 byte digit planes, argmax) "
                               "103424x1024 m=1", "us_per_launch": round(us, 3),
                     "algorithmic_bytes": int(alg),
                     # a bare 16-byte streaming read of the same bytes, timed the same way
                     "stream_read_us": round(stream_us, 3), "frac_of_stream_read": round(stream_us / us, 4)},
        "decode_effective_GB_s": round(per_token_bytes * tok_s / 1e9, 1),
        "cpu_baseline": cpu,
    }
    result.update(extra)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
