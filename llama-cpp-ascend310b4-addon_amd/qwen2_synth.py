"""Random-init Qwen2-shaped models in ggml tensor formats (numpy only).

Used by the benchmark and the tests to stand in for GGUF checkpoints (no model
files exist offline).  Tensors are named as llama.cpp's GGUF loader names them
and laid out as ggml stores them: Q8_0 / Q4_0 block rows for the projections,
an fp16 token embedding that doubles as the tied output head, fp32 norms and
q/k/v biases.  Q8_0 blocks have qs uniform in [-127, 127] and
d = fp16(|N(0, 0.02)| / 127); Q4_0 nibbles are uniform in [0, 15] with
d = fp16(|N(0, 0.02)| / 8); F16 projections are N(0, 0.02).  A8W8 models carry
SmoothQuant factors uniform in [0.5, 2], one vector per projection input (q/k/v share
one, gate/up share one).  With Q8_0 projections the blocks are taken to be the already
smoothed weights W*diag(s); with F16 projections the weights are the unsmoothed W and
the backend folds s in when it quantizes them at upload (GGML_MI355X_A8W8=1).
With random weights, attention scores are small and the softmax is nearly uniform;
qk_gain > 1 scales the q and k projection scales so that attention is peaked and the
logits depend on which positions it selects (RoPE angles, the GQA head map).
"""
import numpy as np

GGML_TYPE_F16 = 1
GGML_TYPE_Q4_0 = 2
GGML_TYPE_Q8_0 = 8


def qwen2_1p5b(n_ctx=576, **kw):
    hp = dict(n_layer=28, n_embd=1536, n_head=12, n_head_kv=2, head_dim=128, n_ff=8960, n_vocab=151936,
              n_ctx=n_ctx, rms_eps=1e-6, rope_theta=1e6, wtype=GGML_TYPE_Q8_0, use_bias=1, n_seq=1)
    hp.update(kw)
    return hp


def qwen2_7b(n_ctx=32768 + 128, **kw):
    hp = dict(n_layer=28, n_embd=3584, n_head=28, n_head_kv=4, head_dim=128, n_ff=18944, n_vocab=152064,
              n_ctx=n_ctx, rms_eps=1e-6, rope_theta=1e6, wtype=GGML_TYPE_Q4_0, use_bias=1, n_seq=1)
    hp.update(kw)
    return hp


def _f16(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def q8_0_rows(rng, n, k):
    nb = k // 32
    blk = np.empty((n, nb, 34), dtype=np.uint8)
    blk[:, :, 2:] = rng.integers(-127, 128, size=(n, nb, 32), dtype=np.int8).view(np.uint8)
    d = _f16(np.abs(rng.standard_normal((n, nb), dtype=np.float32)) * np.float32(0.02 / 127.0))
    blk[:, :, 0:2] = d.view(np.uint8).reshape(n, nb, 2)
    return blk.reshape(n, nb * 34)


def q4_0_rows(rng, n, k):
    nb = k // 32
    blk = np.empty((n, nb, 18), dtype=np.uint8)
    blk[:, :, 2:] = rng.integers(0, 256, size=(n, nb, 16), dtype=np.uint8)  # two uniform nibbles per byte
    d = _f16(np.abs(rng.standard_normal((n, nb), dtype=np.float32)) * np.float32(0.02 / 8.0))
    blk[:, :, 0:2] = d.view(np.uint8).reshape(n, nb, 2)
    return blk.reshape(n, nb * 18)


def f16_rows(rng, n, k):
    return _f16(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))


def projections(hp):
    """(name suffix, n_out, n_in, smoothing group) of one layer's matmul weights"""
    E, F, nkv = hp["n_embd"], hp["n_ff"], hp["n_head_kv"] * hp["head_dim"]
    return (("attn_q", E, E, "attn"), ("attn_k", nkv, E, "attn"), ("attn_v", nkv, E, "attn"),
            ("attn_output", E, E, "o"), ("ffn_gate", F, E, "ffn"), ("ffn_up", F, E, "ffn"),
            ("ffn_down", E, F, "down"))


def _scale_blocks(blk, gain, bsize):
    n = blk.shape[0]
    b = blk.reshape(n, -1, bsize)
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float32) * np.float32(gain)
    b[:, :, 0:2] = d.astype(np.float16).view(np.uint8).reshape(n, -1, 2)
    return b.reshape(n, -1)


def synth(hp, seed=0, smooth=None, qk_gain=1.0):
    """-> (tensors: name -> ggml-format array, smooth: weight name -> s or None)"""
    rng = np.random.default_rng(seed)
    E = hp["n_embd"]
    nkv = hp["n_head_kv"] * hp["head_dim"]
    wt = hp["wtype"]
    if smooth is None:
        smooth = wt in (GGML_TYPE_Q8_0, GGML_TYPE_F16)
    rows = {GGML_TYPE_Q8_0: q8_0_rows, GGML_TYPE_Q4_0: q4_0_rows, GGML_TYPE_F16: f16_rows}[wt]
    t = {"token_embd.weight": _f16(rng.standard_normal((hp["n_vocab"], E), dtype=np.float32) * np.float32(0.02)),
         "output_norm.weight": rng.uniform(0.8, 1.2, E).astype(np.float32)}
    sm = {}
    for il in range(hp["n_layer"]):
        p = f"blk.{il}."
        t[p + "attn_norm.weight"] = rng.uniform(0.8, 1.2, E).astype(np.float32)
        t[p + "ffn_norm.weight"] = rng.uniform(0.8, 1.2, E).astype(np.float32)
        groups = {}
        for name, n, k, grp in projections(hp):
            t[p + name + ".weight"] = rows(rng, n, k)
            if qk_gain != 1.0 and name in ("attn_q", "attn_k"):
                if wt == GGML_TYPE_F16:
                    t[p + name + ".weight"] = _f16(t[p + name + ".weight"].view(np.float16).astype(np.float32) *
                                                   np.float32(qk_gain))
                else:
                    t[p + name + ".weight"] = _scale_blocks(t[p + name + ".weight"], qk_gain,
                                                            34 if wt == GGML_TYPE_Q8_0 else 18)
            if smooth:
                if grp not in groups:
                    groups[grp] = rng.uniform(0.5, 2.0, k).astype(np.float32)
                sm[p + name + ".weight"] = groups[grp]
        if hp.get("use_bias", 1):
            t[p + "attn_q.bias"] = (rng.standard_normal(E) * 0.02).astype(np.float32)
            t[p + "attn_k.bias"] = (rng.standard_normal(nkv) * 0.02).astype(np.float32)
            t[p + "attn_v.bias"] = (rng.standard_normal(nkv) * 0.02).astype(np.float32)
    return t, sm


def weight_bytes(hp):
    """bytes one decode token streams: projection blocks + the fp16 tied head"""
    per = sum(n * k // 32 * (34 if hp["wtype"] == GGML_TYPE_Q8_0 else 18) for _, n, k, _ in projections(hp))
    return hp["n_layer"] * per + hp["n_vocab"] * hp["n_embd"] * 2


def kv_bytes_per_position(hp):
    return hp["n_layer"] * 2 * hp["n_head_kv"] * hp["head_dim"] * 2
