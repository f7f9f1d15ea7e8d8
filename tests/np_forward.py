"""Independent float64 numpy forward pass of the dense Llama decoder, used to
pin the oracle's TransformerRunner restatement (and the HIP runner) on small
models.  Written from the model definition, not from the oracle's code: RMS
norm, interleaved-pair RoPE with theta = pos / base^(2i/hd), causal GQA
attention over the cache, SwiGLU, residuals, final norm and lm_head."""
import numpy as np

import oracle


def dense(t):
    """Dequantized f64 matrix [rows][cols] (or f64 vector) of a model tensor."""
    if t.data.dtype == np.float32:
        return t.data.astype(np.float64)
    cols, rows = t.shape
    return oracle.dequant(int(t.dtype), t.data).astype(np.float64).reshape(rows, cols)


class NpForward:
    def __init__(self, model):
        self.m = model
        c = model.cfg
        self.c = c
        self.W = {k: dense(t) for k, t in model.tensors.items() if k != "token_embd.weight"}
        self.embd = model["token_embd.weight"]
        self.k = [[] for _ in range(c.n_layers)]
        self.v = [[] for _ in range(c.n_layers)]
        self.pos = 0

    def _rms(self, x, w):
        return x / np.sqrt(np.mean(x * x) + self.c.norm_eps) * w

    def _rope(self, v, pos):
        hd = self.c.head_dim
        out = v.copy().reshape(-1, hd)
        i = np.arange(hd // 2)
        th = pos / (self.c.rope_base ** (2.0 * i / hd))
        c, s = np.cos(th), np.sin(th)
        x0, x1 = out[:, 0::2].copy(), out[:, 1::2].copy()
        out[:, 0::2] = x0 * c - x1 * s
        out[:, 1::2] = x0 * s + x1 * c
        return out.reshape(-1)

    def forward(self, token):
        c, W = self.c, self.W
        cols, rows = self.embd.shape
        from yule_amd.formats import row_bytes
        rb = row_bytes(self.embd.dtype, cols)
        h = oracle.dequant(int(self.embd.dtype), self.embd.data[token * rb:(token + 1) * rb]).astype(np.float64)
        hd, g = c.head_dim, c.n_heads // c.n_kv_heads
        for L in range(c.n_layers):
            p = f"blk.{L}."
            x = self._rms(h, W[p + "attn_norm.weight"])
            q = self._rope(W[p + "attn_q.weight"] @ x, self.pos)
            k = self._rope(W[p + "attn_k.weight"] @ x, self.pos)
            v = W[p + "attn_v.weight"] @ x
            self.k[L].append(k)
            self.v[L].append(v)
            K, V = np.stack(self.k[L]), np.stack(self.v[L])
            att = np.zeros(c.n_heads * hd)
            for hh in range(c.n_heads):
                kv = hh // g
                s = K[:, kv * hd:(kv + 1) * hd] @ q[hh * hd:(hh + 1) * hd] / np.sqrt(hd)
                pr = np.exp(s - s.max())
                pr /= pr.sum()
                att[hh * hd:(hh + 1) * hd] = pr @ V[:, kv * hd:(kv + 1) * hd]
            h = h + W[p + "attn_output.weight"] @ att
            x = self._rms(h, W[p + "ffn_norm.weight"])
            gt, up = W[p + "ffn_gate.weight"] @ x, W[p + "ffn_up.weight"] @ x
            h = h + W[p + "ffn_down.weight"] @ (gt / (1.0 + np.exp(-gt)) * up)
        self.pos += 1
        return W["output.weight"] @ self._rms(h, W["output_norm.weight"])
