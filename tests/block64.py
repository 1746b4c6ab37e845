"""Float64 transcription of the DA3-BASE pre-LN ViT block (BASELINE config
3), the exact result of the block on float32 inputs and weights: LN -> QKV
(+bias) -> [late blocks: LayerNorm of each 64-wide Q/K head row] -> 2-D RoPE
on Q, K -> softmax(QK^T/8)V -> out-proj (+bias) * LayerScale + residual ->
LN -> fc1 (+bias) -> exact-erf GELU -> fc2 (+bias) * LayerScale + residual.
It pins the oracle's block (tests/test_oracle_block.py) and measures how
close the oracle and the device come to the exact block
(tests/test_gpu_block.py)."""
import math

import numpy as np

_erf = np.vectorize(math.erf)


def block64(x, w, T, pos, eps=1e-6, freq=100.0):
    D, H = 768, 12
    f = {k: np.asarray(v, np.float64) for k, v in w.items()}
    x = np.asarray(x, np.float64).reshape(T, D)

    def ln(z, g, b):
        mu = z.mean(1, keepdims=True)
        return (z - mu) / np.sqrt(((z - mu) ** 2).mean(1, keepdims=True) + eps) * g + b

    h = ln(x, f["ln1_gamma"], f["ln1_beta"])
    qkv = h @ f["w_qkv"].reshape(D, 3 * D) + f["b_qkv"]
    q, k, v = (qkv[:, i * D:(i + 1) * D].reshape(T, H, 64).transpose(1, 0, 2) for i in range(3))
    if "q_norm_gamma" in f:  # DA3 late block: LayerNorm of each 64-wide head row
        q = ln(q.reshape(-1, 64), f["q_norm_gamma"], f["q_norm_beta"]).reshape(H, T, 64)
        k = ln(k.reshape(-1, 64), f["k_norm_gamma"], f["k_norm_beta"]).reshape(H, T, 64)
    if pos is not None:
        theta = np.float32(freq) ** (-2.0 * np.arange(16) / 32.0)
        p = pos.reshape(T, 2).astype(np.float64)

        def rope(z):
            z = z.copy()
            for ax in range(2):
                ang = p[:, ax][:, None] * theta[None, :]
                s, c = np.sin(ang), np.cos(ang)
                a = z[:, :, ax * 32:ax * 32 + 16].copy()
                b = z[:, :, ax * 32 + 16:ax * 32 + 32].copy()
                z[:, :, ax * 32:ax * 32 + 16] = a * c - b * s
                z[:, :, ax * 32 + 16:ax * 32 + 32] = b * c + a * s
            return z

        q, k = rope(q), rope(k)
    s = q @ k.transpose(0, 2, 1) / 8.0
    pr = np.exp(s - s.max(-1, keepdims=True))
    att = (pr / pr.sum(-1, keepdims=True)) @ v
    att = att.transpose(1, 0, 2).reshape(T, D)
    x = x + (att @ f["w_proj"].reshape(D, D) + f["b_proj"]) * f["ls1"]
    h = ln(x, f["ln2_gamma"], f["ln2_beta"])
    m = h @ f["w_fc1"].reshape(D, 3072) + f["b_fc1"]
    m = 0.5 * m * (1 + _erf(m / math.sqrt(2)))
    x = x + (m @ f["w_fc2"].reshape(3072, D) + f["b_fc2"]) * f["ls2"]
    return x.reshape(-1), att.reshape(-1)
