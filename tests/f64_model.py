"""An independent float64 statement of one Gemma-3 token step, written from
the reference's unfused debug forward pass (debug.html:1983-2087: embedding,
rmsNorm, Q/K/V, per-head norm, RoPE, KV store, scores, softmax, weighted V,
O projection, post-attention norm, residual add, FFN norm, gate/up, GELU*up,
down, post-FFN norm, residual add) rather than from the fused src/ path the
C oracle follows. Vectorised numpy in float64, so it shares neither code
nor rounding with the oracle; used to pin the oracle's composition.
"""
import numpy as np

from gemma_amd.gguf import dequantize_q8_0_np


class F64Model:
    def __init__(self, shape, tensors):
        self.s = shape
        H, I, Q, KV = shape.hidden, shape.inter, shape.q_dim, shape.kv_dim

        def mat(name, rows, k):
            return dequantize_q8_0_np(tensors[name][2], rows * k).astype(np.float64).reshape(rows, k)

        def vec(name):
            return np.asarray(tensors[name][2], dtype=np.float64)

        self.emb = mat("token_embd.weight", shape.vocab, H)
        self.out_norm = vec("output_norm.weight")
        self.L = []
        for l in range(shape.layers):
            p = f"blk.{l}."
            self.L.append(dict(
                q=mat(p + "attn_q.weight", Q, H), k=mat(p + "attn_k.weight", KV, H),
                v=mat(p + "attn_v.weight", KV, H), o=mat(p + "attn_output.weight", H, Q),
                gate=mat(p + "ffn_gate.weight", I, H), up=mat(p + "ffn_up.weight", I, H),
                down=mat(p + "ffn_down.weight", H, I),
                attn_norm=vec(p + "attn_norm.weight"), ffn_norm=vec(p + "ffn_norm.weight"),
                qn=vec(p + "attn_q_norm.weight"), kn=vec(p + "attn_k_norm.weight"),
                post_attn=vec(p + "post_attention_norm.weight"), post_ffw=vec(p + "post_ffw_norm.weight"),
            ))
        self.kc = np.zeros((shape.layers, shape.ctx, KV))
        self.vc = np.zeros((shape.layers, shape.ctx, KV))
        self.hist = np.zeros((shape.layers, H))

    def _norm(self, x, w):
        return x * w / np.sqrt(np.mean(x * x) + self.s.eps)

    def _rope(self, x, pos, theta):
        hd = self.s.head_dim
        half = hd // 2
        i = np.arange(half)
        freq = 1.0 / np.power(np.float64(theta), 2.0 * i / hd)
        # the reference rounds the angle to f32: f32(pos) * f32(freq)
        ang = (np.float32(pos) * freq.astype(np.float32)).astype(np.float64)
        c, s = np.cos(ang), np.sin(ang)
        x = x.reshape(-1, hd)
        a, b = x[:, :half], x[:, half:]
        return np.concatenate([a * c - b * s, a * s + b * c], axis=1)

    def forward(self, token, pos):
        s = self.s
        hd = s.head_dim
        h = self.emb[token] * np.sqrt(s.hidden)
        for l, W in enumerate(self.L):
            swa = (l % s.swa_period) < (s.swa_period - 1)
            theta = s.theta_local if swa else s.theta_global
            lo = max(0, pos - s.window + 1) if (swa and s.window > 0) else 0
            x = self._norm(h, W["attn_norm"])
            q = (W["q"] @ x).reshape(s.n_q, hd)
            k = (W["k"] @ x).reshape(s.n_kv, hd)
            v = W["v"] @ x
            q = np.stack([self._norm(qh, W["qn"]) for qh in q])
            k = np.stack([self._norm(kh, W["kn"]) for kh in k])
            q = self._rope(q, pos, theta)
            k = self._rope(k, pos, theta).reshape(-1)
            self.kc[l, pos] = k
            self.vc[l, pos] = v
            K = self.kc[l, lo:pos + 1]
            V = self.vc[l, lo:pos + 1]
            sc = q @ K.T / np.sqrt(hd)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            att = (p @ V).reshape(-1)
            res = h + self._norm(W["o"] @ att, W["post_attn"])
            x = self._norm(res, W["ffn_norm"])
            g, u = W["gate"] @ x, W["up"] @ x
            t = np.clip(np.sqrt(2 / np.pi) * g * (1 + 0.044715 * g * g), -15, 15)
            act = 0.5 * g * (1 + np.tanh(t)) * u
            h = res + self._norm(W["down"] @ act, W["post_ffw"])
            self.hist[l] = h
        self.hidden = h
        self.normed = self._norm(h, self.out_norm)
        return self.normed

    def logits(self):
        return self.emb @ self.normed
