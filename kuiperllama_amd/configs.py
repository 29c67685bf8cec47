"""Model configurations.

``BASELINE`` holds the five synthetic workloads the benchmark and the parity
tests are defined on (Llama2-110M fp32, Llama-3.2-1B fp32, Llama2-7B int8
g64, Qwen2.5-1.5B fp32 with a 4000-position cache, Qwen3-4B fp32 with a
512-token prompt).  ``TINY`` holds the same architectures at sizes the CPU
oracle runs in milliseconds; every family, RoPE pairing, GQA ratio, tie mode
and the int8 layout is covered.
"""
from __future__ import annotations

from dataclasses import asdict, dataclass, replace

from . import _lib


@dataclass(frozen=True)
class Config:
    name: str
    family: int
    dim: int
    hidden_dim: int
    layers: int
    heads: int
    kv_heads: int
    vocab: int
    seq_len: int
    tied: bool
    q_dim: int = 0  # 0: same as dim (everything but Qwen3)
    group_size: int = 0  # >0: int8 weights, one fp32 scale per group
    prompt_len: int = 16
    decode_steps: int = 128
    norm_std: float = 0.0  # 0: norm weights 1.0; >0: 1 + N(0, norm_std) per norm and layer

    @property
    def qd(self) -> int:
        return self.q_dim or self.dim

    @property
    def head_size(self) -> int:
        return self.qd // self.heads

    @property
    def kv_dim(self) -> int:
        return self.qd * self.kv_heads // self.heads

    @property
    def quant(self) -> bool:
        return self.group_size > 0

    def spec(self) -> _lib.ModelSpec:
        return _lib.ModelSpec(
            family=self.family,
            dim=self.dim,
            q_dim=self.qd,
            hidden_dim=self.hidden_dim,
            layers=self.layers,
            heads=self.heads,
            kv_heads=self.kv_heads,
            vocab=self.vocab,
            seq_len=self.seq_len,
            tied=int(self.tied),
            group_size=self.group_size,
            norm_stddev=self.norm_std,
        )

    def with_(self, **kw) -> "Config":
        return replace(self, **kw)

    def as_dict(self) -> dict:
        return asdict(self)

    # --- algorithmic bytes per decode token (HBM roofline) ---------------
    def weight_bytes_per_token(self) -> int:
        """Bytes of every weight a decode step streams: the 7 projections of
        every layer, the classifier, the norm vectors (and Qwen2 biases,
        Qwen3 q/k norms).  The embedding row gather (dim floats) is counted
        too; a tied classifier is the embedding matrix, counted once."""
        D, Dq, Dkv, F, L, V = self.dim, self.qd, self.kv_dim, self.hidden_dim, self.layers, self.vocab
        mats = L * (Dq * D + 2 * Dkv * D + D * Dq + 3 * F * D) + V * D
        if self.quant:
            mat_bytes = mats + (mats // self.group_size) * 4
        else:
            mat_bytes = mats * 4
        vec = (2 * L + 1) * D + D  # norms + embedding row
        if self.family == _lib.FAMILY_QWEN2:
            vec += L * (Dq + 2 * Dkv)
        if self.family == _lib.FAMILY_QWEN3:
            vec += 2 * L * self.head_size
        return mat_bytes + vec * 4

    def kv_bytes_per_token(self, pos: int) -> int:
        """K and V rows read at position pos (pos + 1 positions, every layer)
        plus the new row written."""
        return 2 * self.layers * self.kv_dim * 4 * (pos + 1) + 2 * self.layers * self.kv_dim * 4

    def prefill_flops(self, n: int) -> int:
        """Algorithmic FLOPs of a batched prefill of positions 0 .. n-1: the
        seven projections of every layer on n rows (2 flops per weight per
        row), causal attention (q.k and p.v over t <= position: 4 * heads *
        head_size * (pos + 1) per position and layer) and the classifier of
        the last position."""
        return sum(self.prefill_flops_parts(n))

    def prefill_flops_parts(self, n: int):
        """prefill_flops as (projections, attention, classifier)."""
        D, Dq, Dkv, F, L = self.dim, self.qd, self.kv_dim, self.hidden_dim, self.layers
        proj = L * (Dq * D + 2 * Dkv * D + D * Dq + 3 * F * D)
        attn = L * 4 * self.heads * self.head_size * (n * (n + 1) // 2)
        return 2 * proj * n, attn, 2 * self.vocab * D

    def decode_bytes(self, first_pos: int, steps: int) -> int:
        """Algorithmic HBM bytes of `steps` decode steps at positions
        first_pos .. first_pos + steps - 1."""
        w = self.weight_bytes_per_token()
        return sum(w + self.kv_bytes_per_token(p) for p in range(first_pos, first_pos + steps))


L2, L3, Q2, Q3 = _lib.FAMILY_LLAMA2, _lib.FAMILY_LLAMA3, _lib.FAMILY_QWEN2, _lib.FAMILY_QWEN3

BASELINE = {
    "llama2_110m": Config("llama2_110m", L2, 768, 2048, 12, 12, 12, 32000, 1024, False,
                          prompt_len=16, decode_steps=128),
    "llama32_1b": Config("llama32_1b", L3, 2048, 8192, 16, 32, 8, 128256, 1024, True,
                         prompt_len=64, decode_steps=256),
    "llama2_7b_q8": Config("llama2_7b_q8", L2, 4096, 11008, 32, 32, 32, 32000, 1024, False,
                           group_size=64, prompt_len=32, decode_steps=128),
    "qwen25_15b": Config("qwen25_15b", Q2, 1536, 8960, 28, 12, 2, 151936, 4096, True,
                         prompt_len=4000, decode_steps=96),
    "qwen3_4b": Config("qwen3_4b", Q3, 2560, 9728, 36, 32, 8, 151936, 1024, False, q_dim=4096,
                       prompt_len=512, decode_steps=128),
}

TINY = {
    "tiny_llama2": Config("tiny_llama2", L2, 128, 256, 2, 4, 4, 512, 64, False, norm_std=0.1,
                          prompt_len=5, decode_steps=20),
    "tiny_llama3": Config("tiny_llama3", L3, 256, 512, 2, 4, 2, 1000, 96, True, norm_std=0.1,
                          prompt_len=7, decode_steps=40),
    "tiny_q8": Config("tiny_q8", L2, 256, 512, 2, 2, 2, 1024, 64, False, group_size=64, norm_std=0.1,
                      prompt_len=4, decode_steps=20),
    "tiny_qwen2": Config("tiny_qwen2", Q2, 256, 384, 2, 2, 1, 777, 128, True, norm_std=0.1,
                         prompt_len=9, decode_steps=40),
    "tiny_qwen2_q8": Config("tiny_qwen2_q8", Q2, 256, 384, 2, 4, 2, 768, 64, False, group_size=64,
                            norm_std=0.1, prompt_len=5, decode_steps=20),
    "tiny_qwen3": Config("tiny_qwen3", Q3, 192, 320, 2, 4, 2, 640, 64, False, q_dim=256, norm_std=0.1,
                         prompt_len=6, decode_steps=20),
}

ALL = {**BASELINE, **TINY}
