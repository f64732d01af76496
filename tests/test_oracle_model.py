"""The CPU Qwen2 decode restatement (oracle/qwen2_oracle.c) against an independent
float64 numpy transformer written from the textbook formulas.

The numpy model dequantizes the weights and then computes in float64 without any of
ggml's roundings (no activation quantization, no fp16 KV cache, no fp16 accumulator):
RMSNorm, RoPE in the NeoX half-split pairing with theta_i = pos * base^(-2i/d) taken in
closed form, grouped-query softmax attention (query head h reads KV head
h // (n_head / n_head_kv)), SwiGLU, residuals, final norm, tied head.  The two differ
by ggml's rounding only (measured: Q4_0 with fp16 activations 1.4e-4 of the logit
scale, Q8_0 with per-block int8 activations 2.8e-3), while a wiring mistake -- a dropped bias or
residual, adjacent instead of half-split RoPE pairs, a wrong GQA map, a missing
SmoothQuant reciprocal -- moves them by 5e-2 or more (attention made peaked by
qk_gain so that RoPE angles and the head map matter).  One test plants
such mistakes in the numpy model to show the bar separates them.
"""
import numpy as np
import pytest

import qwen2_synth as qs


def _deq(t, typ, n, k):
    nb = k // 32
    if typ == qs.GGML_TYPE_Q8_0:
        b = t.reshape(n, nb, 34)
        d = b[:, :, 0:2].copy().view(np.float16).astype(np.float64)
        q = b[:, :, 2:].view(np.int8).astype(np.float64)
        return (q * d).reshape(n, k)
    b = t.reshape(n, nb, 18)
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float64)
    qs_ = b[:, :, 2:]
    lo = (qs_ & 0x0F).astype(np.float64) - 8.0
    hi = (qs_ >> 4).astype(np.float64) - 8.0
    return (np.concatenate([lo, hi], axis=2) * d).reshape(n, k)


class NumpyQwen2:
    def __init__(self, hp, tensors, smooth, plant=None):
        self.hp, self.plant = hp, plant or set()
        E, hd = hp["n_embd"], hp["head_dim"]
        self.emb = tensors["token_embd.weight"].view(np.float16).astype(np.float64).reshape(hp["n_vocab"], E)
        self.onorm = tensors["output_norm.weight"].astype(np.float64)
        self.layers = []
        for il in range(hp["n_layer"]):
            p = f"blk.{il}."
            L = {"attn_norm": tensors[p + "attn_norm.weight"].astype(np.float64),
                 "ffn_norm": tensors[p + "ffn_norm.weight"].astype(np.float64)}
            for name, n, k, _ in qs.projections(hp):
                w = _deq(tensors[p + name + ".weight"], hp["wtype"], n, k)
                s = smooth.get(p + name + ".weight") if smooth else None
                if s is not None and "no_smooth" not in self.plant:
                    w = w / np.asarray(s, np.float64)[None, :]   # blocks hold W*diag(s)
                L[name] = w
            for b in ("attn_q", "attn_k", "attn_v"):
                t = tensors.get(p + b + ".bias")
                L[b + ".bias"] = None if t is None or "no_bias" in self.plant else t.astype(np.float64)
            self.layers.append(L)
        self.kc = [[] for _ in range(hp["n_layer"])]
        self.vc = [[] for _ in range(hp["n_layer"])]

    def _rope(self, x, pos):
        hd = self.hp["head_dim"]
        i = np.arange(hd // 2, dtype=np.float64)
        th = pos * self.hp["rope_theta"] ** (-2.0 * i / hd)
        c, s = np.cos(th), np.sin(th)
        if "adjacent_rope" in self.plant:
            a, b = x[:, 0::2].copy(), x[:, 1::2].copy()
            out = np.empty_like(x)
            out[:, 0::2], out[:, 1::2] = a * c - b * s, a * s + b * c
            return out
        a, b = x[:, : hd // 2], x[:, hd // 2:]
        return np.concatenate([a * c - b * s, a * s + b * c], axis=1)

    def _norm(self, x, w):
        return x / np.sqrt(np.mean(x * x) + self.hp["rms_eps"]) * w

    def decode(self, token, pos):
        hp = self.hp
        nh, nkv, hd = hp["n_head"], hp["n_head_kv"], hp["head_dim"]
        x = self.emb[token].copy()
        for il, L in enumerate(self.layers):
            h = self._norm(x, L["attn_norm"])
            q, k, v = L["attn_q"] @ h, L["attn_k"] @ h, L["attn_v"] @ h
            if L["attn_q.bias"] is not None:
                q, k, v = q + L["attn_q.bias"], k + L["attn_k.bias"], v + L["attn_v.bias"]
            q = self._rope(q.reshape(nh, hd), pos)
            k = self._rope(k.reshape(nkv, hd), pos)
            self.kc[il].append(k)
            self.vc[il].append(v.reshape(nkv, hd))
            K, V = np.stack(self.kc[il]), np.stack(self.vc[il])   # [pos+1, nkv, hd]
            att = np.empty((nh, hd))
            for hq in range(nh):
                hk = hq % nkv if "gqa_modulo" in self.plant else hq // (nh // nkv)
                sc = K[:, hk, :] @ q[hq] / np.sqrt(hd)
                p_ = np.exp(sc - sc.max())
                att[hq] = (p_ / p_.sum()) @ V[:, hk, :]
            o = L["attn_output"] @ att.reshape(-1)
            x = x + o
            h = self._norm(x, L["ffn_norm"])
            g, u = L["ffn_gate"] @ h, L["ffn_up"] @ h
            o = L["ffn_down"] @ (g / (1.0 + np.exp(-g)) * u)
            x = o if "no_ffn_residual" in self.plant else x + o
        h = self._norm(x, self.onorm)
        return self.emb @ h


QK_GAIN = 6.0   # peaked attention: the logits depend on the RoPE angles and the head map


def _tiny(wtype):
    return qs.qwen2_1p5b(n_layer=2, n_embd=128, n_head=4, n_head_kv=2, head_dim=32, n_ff=256, n_vocab=300,
                         n_ctx=32, wtype=wtype)


def _max_rel(orc, hp, plant=None, n_pos=16, seed=11):
    tensors, smooth = qs.synth(hp, seed=seed, qk_gain=QK_GAIN)
    cpu = orc.Qwen2(hp, tensors, smooth, fa_mode=1, n_threads=2)
    ref = NumpyQwen2(hp, tensors, smooth, plant)
    rng = np.random.default_rng(seed)
    worst = 0.0
    for pos, tok in enumerate(rng.integers(0, hp["n_vocab"], n_pos)):
        _, lc = cpu.decode(int(tok), pos)
        lr = ref.decode(int(tok), pos)
        worst = max(worst, float(np.abs(lc - lr).max() / np.abs(lr).max()))
    return worst


BAR = {qs.GGML_TYPE_Q4_0: 1e-3, qs.GGML_TYPE_Q8_0: 1e-2}


@pytest.mark.parametrize("wtype", [qs.GGML_TYPE_Q4_0, qs.GGML_TYPE_Q8_0])
def test_qwen2_oracle_matches_float64_transformer(orc, wtype):
    assert _max_rel(orc, _tiny(wtype)) < BAR[wtype]


@pytest.mark.parametrize("plant", ["adjacent_rope", "gqa_modulo", "no_bias", "no_ffn_residual", "no_smooth"])
def test_planted_wiring_mistakes_exceed_the_bar(orc, plant):
    wtype = qs.GGML_TYPE_Q8_0 if plant == "no_smooth" else qs.GGML_TYPE_Q4_0
    assert _max_rel(orc, _tiny(wtype), {plant}) > 5 * BAR[wtype]
