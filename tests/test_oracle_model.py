"""The oracle's whole decoder step and generation loop against the float64
numpy decoder, including the Q4/Q6 residual behaviour."""
import numpy as np
import pytest

from rapidocrvl_amd import synth
from rapidocrvl_amd.config import DecoderConfig

from decoder_f64 import DecoderF64

Q8, Q4, Q6 = 1000, 1001, 1002
TINY = DecoderConfig(hidden=128, inter=192, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=300, eps=1e-5,
                     rope_theta=500000.0)


@pytest.fixture(scope="module", params=[Q8, Q4, Q6], ids=["q8", "q4", "q6"])
def tiny(request):
    return request.param, synth.make_weights(TINY, request.param, seed=3)


def _oracle_model(orc, weights, quirk=True):
    m = orc.Model(TINY)
    m.load_weights(weights)
    m.set_quirk(quirk)
    return m


@pytest.mark.parametrize("quirk", [True, False])
def test_step_logits_match_f64(orc, tiny, quirk):
    qtype, w = tiny
    m = _oracle_model(orc, w, quirk)
    ref = DecoderF64(TINY, w, quirk=quirk)
    s = m.seq(16)
    for p in range(10):  # covers the first-token, 1..5 and >=6 branches
        emb = w["embed"][(7 * p + 3) % TINY.vocab]
        tok, logits, _ = s.step(emb, (p, p, p))
        want = ref.step(emb, (p, p, p))
        assert np.max(np.abs(logits - want)) < 2e-4 * max(1.0, np.max(np.abs(want))), (p, qtype)
        assert tok == int(np.argmax(logits))


def test_quirk_changes_residual_only_for_q4_q6(orc, tiny):
    qtype, w = tiny
    on, off = _oracle_model(orc, w, True), _oracle_model(orc, w, False)
    s_on, s_off = on.seq(4), off.seq(4)
    emb = w["embed"][5]
    _, l_on, _ = s_on.step(emb, (0, 0, 0))
    _, l_off, _ = s_off.step(emb, (0, 0, 0))
    if qtype == Q8:
        assert np.array_equal(l_on, l_off)
    else:
        assert np.max(np.abs(l_on - l_off)) > 1e-3


def test_non_final_prompt_token_only_appends(orc, tiny):
    qtype, w = tiny
    m = _oracle_model(orc, w)
    a, b = m.seq(8), m.seq(8)
    e0, e1 = w["embed"][1], w["embed"][2]
    a.step(e0, (0, 0, 0), need_logits=False)
    b.step(e0, (0, 0, 0), need_logits=True)
    for li in range(TINY.layers):
        ka, va = a.kv(li)
        kb, vb = b.kv(li)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    _, la, _ = a.step(e1, (1, 1, 1))
    _, lb, _ = b.step(e1, (1, 1, 1))
    assert np.array_equal(la, lb)


def test_kv_rows_follow_append_order(orc, tiny):
    # kvCache.append: row t = t-th token, K after RoPE, V raw (model.go:5593-5634)
    qtype, w = tiny
    m = _oracle_model(orc, w)
    ref = DecoderF64(TINY, w)
    s = m.seq(8)
    for p in range(5):
        emb = w["embed"][p + 10]
        s.step(emb, (p, p, p))
        ref.step(emb, (p, p, p))
    for li in range(TINY.layers):
        k, v = s.kv(li)
        assert k.size == 5 * TINY.kv_rows
        assert np.allclose(k.reshape(5, -1), np.array(ref.k[li]), atol=1e-4)
        assert np.allclose(v.reshape(5, -1), np.array(ref.v[li]), atol=1e-4)


def test_generate_equals_step_loop(orc, tiny):
    qtype, w = tiny
    m = _oracle_model(orc, w)
    ids = np.array([5, 17, 250, 3, 99, 42, 7], np.int32)
    got = m.generate(ids, 9, eos=())
    s = m.seq(32)
    for p, t in enumerate(ids):
        tok, _, _ = s.step(w["embed"][t], (p, p, p), need_logits=p == len(ids) - 1)
    want = [tok]
    for i in range(8):
        p = len(ids) + i
        tok, _, _ = s.step(w["embed"][want[-1]], (p, p, p))
        want.append(tok)
    assert list(got) == want


def test_generate_with_image_positions(orc, tiny):
    qtype, w = tiny
    m = _oracle_model(orc, w)
    IMG = 299
    ids = np.array([5, 6, 7] + [IMG] * 6 + [8, 9], np.int32)
    img = synth.image_embeds(6, TINY.hidden, seed=1) * 0.02
    got = m.generate(ids, 5, eos=(), image_embeds=img, image_token_id=IMG, grid=(1, 4, 6))
    pos, delta = orc.mm_positions(ids, IMG, (1, 4, 6))
    ref = DecoderF64(TINY, w)
    j = 0
    for p, t in enumerate(ids):
        if t == IMG:
            e = img[j]
            j += 1
        else:
            e = w["embed"][t]
        logits = ref.step(e, tuple(pos[p]), need_logits=p == len(ids) - 1)
    want = [int(np.argmax(logits))]
    for i in range(4):
        pp = len(ids) + i + delta
        want.append(int(np.argmax(ref.step(w["embed"][want[-1]], (pp, pp, pp)))))
    assert list(got) == want


def test_eos_stops_generation(orc, tiny):
    qtype, w = tiny
    m = _oracle_model(orc, w)
    ids = np.array([1, 2, 3], np.int32)
    full = m.generate(ids, 6, eos=())
    stop = m.generate(ids, 6, eos=(int(full[2]),))
    first = list(full).index(full[2])
    assert list(stop) == list(full[:first + 1])
