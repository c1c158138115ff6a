"""Independent float64 numpy GPT-2 forward, used only to pin the oracle.

Written from the GPT-2 mathematics (pre-LN blocks, causal softmax attention
scaled by 1/sqrt(head_dim), gelu_new, tied LM head), not from the oracle's
code: a dropped term, a wrong sign or a transposed operand in the oracle makes
the two disagree far beyond float32 rounding.
"""
import numpy as np


def layer_norm(x, w, b, eps):
    x = np.asarray(x, np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def gelu_new(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def attention(q, k, v, n_head, q_pos=None):
    """q [Tq, d], k/v [Tk, d]; query i sits at absolute position q_pos[i]."""
    Tq, d = q.shape
    Tk = k.shape[0]
    hd = d // n_head
    if q_pos is None:
        q_pos = np.arange(Tk - Tq, Tk)
    out = np.zeros((Tq, d))
    mask = np.arange(Tk)[None, :] > np.asarray(q_pos)[:, None]
    for h in range(n_head):
        sl = slice(h * hd, (h + 1) * hd)
        s = q[:, sl] @ k[:, sl].T / np.sqrt(hd)
        s = np.where(mask, -np.inf, s)
        s = s - s.max(-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(-1, keepdims=True)
        out[:, sl] = p @ v[:, sl]
    return out


def forward(sd, ids, n_layer, n_head, eps=1e-5, pos0=0):
    g = {k: np.asarray(v, np.float64) for k, v in sd.items()}
    ids = np.asarray(ids)
    T = ids.size
    x = g["wte.weight"][ids] + g["wpe.weight"][pos0:pos0 + T]
    d = x.shape[1]
    for i in range(n_layer):
        p = f"h.{i}."
        h = layer_norm(x, g[p + "ln_1.weight"], g[p + "ln_1.bias"], eps)
        qkv = h @ g[p + "attn.c_attn.weight"] + g[p + "attn.c_attn.bias"]
        q, k, v = qkv[:, :d], qkv[:, d:2 * d], qkv[:, 2 * d:]
        a = attention(q, k, v, n_head)
        x = x + (a @ g[p + "attn.c_proj.weight"] + g[p + "attn.c_proj.bias"])
        h = layer_norm(x, g[p + "ln_2.weight"], g[p + "ln_2.bias"], eps)
        f = gelu_new(h @ g[p + "mlp.c_fc.weight"] + g[p + "mlp.c_fc.bias"])
        x = x + (f @ g[p + "mlp.c_proj.weight"] + g[p + "mlp.c_proj.bias"])
    x = layer_norm(x, g["ln_f.weight"], g["ln_f.bias"], eps)
    return x @ g["wte.weight"].T
