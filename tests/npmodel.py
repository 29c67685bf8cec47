"""Independent fp64 numpy restatement of the reference decode step, used only to
pin the C++ oracle.

It does not parse the model image: every weight is rebuilt from the
generator's per-tensor normal stream (role, layer), so a wrong offset in the
oracle's image parsing, a misplaced norm/bias/RoPE, a wrong GQA mapping or a
wrong family constant shows up as a logits mismatch.  Family constants cite
the reference: RoPE pairing and theta (kernels/cpu/rope_kernel.cpp:3-122),
eps (kernels/cpu/rmsnorm_kernel.cpp:24-28), q/k norm eps
(kernels/cuda/rmsnorm_kernel.cu:148), Qwen2 bias (op/matmul.cpp:74-77),
Qwen3 q/k norm order (model/qwen3.cpp:485-500).  Norm weights are read per
role and layer: attention norm of layer l, ffn norm of layer l, the final
norm (the reference's rmsnorm_layers_[l], [L + l], [2L], llama3.cpp:599-608,
:687, :723) and Qwen3's q/k norms ([2L + 1 + l], [3L + 1 + l],
qwen3.cpp:485-500).
"""
from __future__ import annotations

import numpy as np

# synth.cpp roles
EMB, WQ, WK, WV, WO, W1, W2, W3, CLS, BQ, BK, BV = range(1, 13)
RMS_ATT, RMS_FFN, RMS_FINAL, Q_NORM, K_NORM = range(13, 18)

FAMILY = {
    0: dict(style="interleaved", theta=1e4, eps=1e-5, bias=False, qknorm=False),
    1: dict(style="half", theta=5e5, eps=1e-5, bias=False, qknorm=False),
    2: dict(style="half", theta=1e6, eps=1e-6, bias=True, qknorm=False),
    3: dict(style="half", theta=1e6, eps=1e-6, bias=False, qknorm=True),
}


class NpModel:
    def __init__(self, K, cfg, seed=1234, stddev=0.02):
        self.cfg = cfg
        f = FAMILY[cfg.family]
        self.f = f
        D, Dq, Dkv, F, L, V = cfg.dim, cfg.qd, cfg.kv_dim, cfg.hidden_dim, cfg.layers, cfg.vocab

        def mat(role, layer, rows, cols):
            w = K.synth_normal(seed, role, layer, rows * cols, stddev)
            if cfg.quant:
                q, s = K.quantize_q8(w, cfg.group_size)
                w = (np.repeat(s, cfg.group_size) * q.astype(np.float32)).astype(np.float32)
            return w.astype(np.float64).reshape(rows, cols)

        def vec(role, layer, n):
            return K.synth_normal(seed, role, layer, n, stddev).astype(np.float64)

        def norm(role, layer, n):
            if not cfg.norm_std:
                return np.ones(n)
            return 1.0 + K.synth_normal(seed, role, layer, n, cfg.norm_std).astype(np.float64)

        self.E = K.synth_normal(seed, EMB, 0, V * D, stddev).astype(np.float64).reshape(V, D)
        self.layers = []
        for l in range(L):
            d = dict(wq=mat(WQ, l, Dq, D), wk=mat(WK, l, Dkv, D), wv=mat(WV, l, Dkv, D),
                     wo=mat(WO, l, D, Dq), w1=mat(W1, l, F, D), w2=mat(W2, l, D, F),
                     w3=mat(W3, l, F, D), rms_att=norm(RMS_ATT, l, D), rms_ffn=norm(RMS_FFN, l, D))
            if f["qknorm"]:
                hd = cfg.head_size
                d.update(q_norm=norm(Q_NORM, l, hd), k_norm=norm(K_NORM, l, hd))
            if f["bias"] and not cfg.quant:
                d.update(bq=vec(BQ, l, Dq), bk=vec(BK, l, Dkv), bv=vec(BV, l, Dkv))
            self.layers.append(d)
        self.rms_final = norm(RMS_FINAL, 0, D)
        self.cls = self.E if (cfg.tied and cfg.family != 3) else mat(CLS, 0, V, D)
        self.kc = np.zeros((L, cfg.seq_len, Dkv))
        self.vc = np.zeros((L, cfg.seq_len, Dkv))

    @staticmethod
    def _rms(x, eps, w):
        return w * (x / np.sqrt(np.mean(x * x) + eps))

    def _rope(self, v, pos, n_heads):
        hd = self.cfg.head_size
        v = v.reshape(n_heads, hd).copy()
        j = np.arange(hd // 2)
        ang = pos * self.f["theta"] ** (-(2.0 * j) / hd)
        c, s = np.cos(ang), np.sin(ang)
        if self.f["style"] == "half":
            a, b = v[:, : hd // 2].copy(), v[:, hd // 2 :].copy()
            v[:, : hd // 2], v[:, hd // 2 :] = a * c - b * s, a * s + b * c
        else:
            a, b = v[:, 0::2].copy(), v[:, 1::2].copy()
            v[:, 0::2], v[:, 1::2] = a * c - b * s, a * s + b * c
        return v.ravel()

    def step(self, token, pos):
        cfg, f = self.cfg, self.f
        H, KVH, hd = cfg.heads, cfg.kv_heads, cfg.head_size
        x = self.E[token].copy()
        for l, w in enumerate(self.layers):
            xb = self._rms(x, f["eps"], w["rms_att"])
            q, k, v = w["wq"] @ xb, w["wk"] @ xb, w["wv"] @ xb
            if "bq" in w:
                q, k, v = q + w["bq"], k + w["bk"], v + w["bv"]
            if f["qknorm"]:
                q = np.concatenate([self._rms(h, 1e-6, w["q_norm"]) for h in q.reshape(H, hd)])
                k = np.concatenate([self._rms(h, 1e-6, w["k_norm"]) for h in k.reshape(KVH, hd)])
            q, k = self._rope(q, pos, H), self._rope(k, pos, KVH)
            self.kc[l, pos], self.vc[l, pos] = k, v
            o = np.empty(H * hd)
            for h in range(H):
                g = h // (H // KVH)
                Kt = self.kc[l, : pos + 1, g * hd : (g + 1) * hd]
                Vt = self.vc[l, : pos + 1, g * hd : (g + 1) * hd]
                s = Kt @ q[h * hd : (h + 1) * hd] / np.sqrt(hd)
                p = np.exp(s - s.max())
                p /= p.sum()
                o[h * hd : (h + 1) * hd] = p @ Vt
            x = x + w["wo"] @ o
            xb = self._rms(x, f["eps"], w["rms_ffn"])
            a, b = w["w1"] @ xb, w["w3"] @ xb
            x = x + w["w2"] @ (a / (1.0 + np.exp(-a)) * b)
        return self.cls @ self._rms(x, f["eps"], self.rms_final)
