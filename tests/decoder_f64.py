"""Float64 numpy decoder written from the layer flow of the reference CPU path
(internal/model/model.go:3475-3643, 3850-4066, 5714-5800), used to pin the
oracle's composition of its pieces.  Exact exp/sqrt; dequantised weights are
codes·scale in f64."""
import math

import numpy as np

from rapidocrvl_amd import lib

Q8, Q4, Q6 = 1000, 1001, 1002


def dequant(entry):
    qt, sc, data, cols = entry
    return lib.unpack_rows(qt, data, cols).astype(np.float64) * sc.astype(np.float64)[:, None], qt


class DecoderF64:
    def __init__(self, cfg, weights, quirk=True):
        self.cfg, self.quirk = cfg, quirk
        self.layers = []
        for lw in weights["layers"]:
            d = {r: dequant(lw[r]) for r in ("q", "k", "v", "o", "gate", "up", "down")}
            d["ln1"] = lw["ln1"].astype(np.float64)
            d["ln2"] = lw["ln2"].astype(np.float64)
            self.layers.append(d)
        self.lm = dequant(weights["lm_head"])[0]
        self.final = weights["final_norm"].astype(np.float64)
        self.embed = weights["embed"]
        half = cfg.head_dim // 2
        self.freq = cfg.rope_theta ** (-np.arange(0, cfg.head_dim, 2) / cfg.head_dim)
        sec = np.cumsum(cfg.mrope_section)
        self.axis = np.minimum(np.searchsorted(sec, np.arange(half), side="right"), 2)
        self.reset()

    def reset(self):
        self.k = [[] for _ in self.layers]
        self.v = [[] for _ in self.layers]

    def rms(self, x, w):
        return x / math.sqrt(np.mean(x * x) + self.cfg.eps) * w

    def rope(self, x, heads, pos):
        if not any(pos):
            return x
        d = self.cfg.head_dim
        half = d // 2
        ang = np.array(pos)[self.axis] * self.freq
        c, s = np.cos(ang), np.sin(ang)
        x = x.reshape(heads, d).copy()
        a, b = x[:, :half].copy(), x[:, half:].copy()
        x[:, :half] = a * c - b * s
        x[:, half:] = b * c + a * s
        return x.reshape(-1)

    def attend(self, q, li):
        cfg = self.cfg
        K = np.array(self.k[li]).reshape(len(self.k[li]), cfg.kv_heads, cfg.head_dim)
        V = np.array(self.v[li]).reshape(len(self.v[li]), cfg.kv_heads, cfg.head_dim)
        g = cfg.heads // cfg.kv_heads
        out = np.zeros(cfg.q_rows)
        scale = float(np.float32(1 / math.sqrt(cfg.head_dim)))
        for h in range(cfg.heads):
            s = K[:, h // g] @ q[h * cfg.head_dim:(h + 1) * cfg.head_dim] * scale
            p = np.exp(s - s.max())
            p /= p.sum()
            out[h * cfg.head_dim:(h + 1) * cfg.head_dim] = p @ V[:, h // g]
        return out

    def step(self, emb, pos, need_logits=True):
        cfg = self.cfg
        h = np.array(emb, np.float64)
        clen = len(self.k[0])
        fn = None
        for li, L in enumerate(self.layers):
            last = li + 1 == len(self.layers)
            x = self.rms(h, L["ln1"])
            k = self.rope(L["k"][0] @ x, cfg.kv_heads, pos)
            v = L["v"][0] @ x
            self.k[li].append(k)
            self.v[li].append(v)
            if last and not need_logits:
                return None
            oq = L["o"][1]
            outonly = self.quirk and oq in (Q4, Q6)
            if clen == 0:
                head_out = np.repeat(v.reshape(cfg.kv_heads, cfg.head_dim), cfg.heads // cfg.kv_heads, axis=0)
                head_out = head_out.reshape(-1)
                in_place = not outonly
            else:
                q = self.rope(L["q"][0] @ x, cfg.heads, pos)
                head_out = self.attend(q, li)
                in_place = (clen + 1 <= 6) or not outonly
            vv = h + L["o"][0] @ head_out
            xn = self.rms(vv, L["ln2"])
            if in_place:
                h = vv
            gg = L["gate"][0] @ xn
            g = gg / (1 + np.exp(-gg)) * (L["up"][0] @ xn)
            if not last:
                h = h + L["down"][0] @ g
            else:
                fn = self.rms(h + L["down"][0] @ g, self.final)
        return self.lm @ fn
