"""Synthetic Llama-family models for the decode runner.

Tensor names follow GGUF / Yule's weight loader (yule-infer/src/
weight_loader.rs:158-199): token_embd.weight, blk.N.{attn_norm, attn_q,
attn_k, attn_v, attn_output, ffn_norm, ffn_gate, ffn_up, ffn_down}.weight,
output_norm.weight, output.weight; GGUF shapes are [cols, rows].

Weights: N(0, 0.02) from per-tensor seeds, quantized by yule_amd.synth.
Norm weights: 1 + N(0, 0.02) in F32.  "Q4_K_M" puts Q6_K on output.weight
and every ffn_down and Q4_K on all other matrices.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass, field

import numpy as np

from . import synth
from .formats import DType, matrix_bytes


@dataclass(frozen=True)
class LlamaConfig:
    n_layers: int
    dim: int
    n_heads: int
    n_kv_heads: int
    ff_dim: int
    vocab: int
    max_seq: int
    norm_eps: float = 1e-5
    rope_base: float = 10000.0

    @property
    def head_dim(self) -> int:
        return self.dim // self.n_heads


# TinyLlama-1.1B shapes, 128-token prompt + 256 decode steps
TINYLLAMA = LlamaConfig(n_layers=22, dim=2048, n_heads=32, n_kv_heads=4, ff_dim=5632, vocab=32000, max_seq=384)
# a small model of the same structure for quick parity runs
TINY_TEST = LlamaConfig(n_layers=2, dim=256, n_heads=8, n_kv_heads=2, ff_dim=512, vocab=1024, max_seq=64)


@dataclass
class Tensor:
    name: str
    dtype: DType
    shape: tuple          # GGUF order: (cols, rows) for matrices, (n,) for vectors
    data: np.ndarray = field(repr=False)


LAYER_KEYS = ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm", "ffn_gate", "ffn_up", "ffn_down")


def quant_scheme(name: str, scheme: str) -> DType:
    if scheme == "Q4_K_M":
        return DType.Q6_K if (name == "output.weight" or name.endswith("ffn_down.weight")) else DType.Q4_K
    return DType[scheme]


class SyntheticModel:
    def __init__(self, cfg: LlamaConfig, tensors: dict[str, Tensor], scheme: str, seed: int):
        self.cfg, self.tensors, self.scheme, self.seed = cfg, tensors, scheme, seed

    def __getitem__(self, name: str) -> Tensor:
        return self.tensors[name]

    def layer(self, i: int) -> dict[str, Tensor]:
        return {k: self.tensors[f"blk.{i}.{k}.weight"] for k in LAYER_KEYS}

    @property
    def weight_bytes(self) -> int:
        return sum(t.data.nbytes for t in self.tensors.values())

    def bytes_per_token(self) -> int:
        """Weight bytes one decode step reads: every matrix except the
        embedding table (one row), plus the norms."""
        c = self.cfg
        embd = self.tensors["token_embd.weight"]
        return self.weight_bytes - embd.data.nbytes + matrix_bytes(embd.dtype, 1, c.dim)

    def to_gguf(self, path, arch: str = "llama") -> int:
        """Write the model as a GGUF v3 file (llama.* metadata, GGUF tensor
        names and [cols, rows] shapes); returns the data-section offset."""
        from .gguf import TensorEntry, model_metadata, write_gguf
        ents = [TensorEntry(t.name, int(t.dtype), tuple(t.shape), t.data) for t in self.tensors.values()]
        return write_gguf(path, model_metadata(self.cfg, arch, f"synthetic-{self.scheme}-{self.seed}"), ents)

    def digest(self) -> str:
        h = hashlib.sha256()
        for name in sorted(self.tensors):
            h.update(name.encode())
            h.update(np.ascontiguousarray(self.tensors[name].data).view(np.uint8))
        return h.hexdigest()

    @classmethod
    def generate(cls, cfg: LlamaConfig, seed: int = 0, scheme: str = "Q4_K_M") -> "SyntheticModel":
        c = cfg
        qd, kvd = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
        specs = [("token_embd.weight", c.vocab, c.dim)]
        for i in range(c.n_layers):
            p = f"blk.{i}."
            specs += [(p + "attn_norm.weight", None, c.dim), (p + "attn_q.weight", qd, c.dim),
                      (p + "attn_k.weight", kvd, c.dim), (p + "attn_v.weight", kvd, c.dim),
                      (p + "attn_output.weight", c.dim, qd), (p + "ffn_norm.weight", None, c.dim),
                      (p + "ffn_gate.weight", c.ff_dim, c.dim), (p + "ffn_up.weight", c.ff_dim, c.dim),
                      (p + "ffn_down.weight", c.dim, c.ff_dim)]
        specs += [("output_norm.weight", None, c.dim), ("output.weight", c.vocab, c.dim)]
        tensors = {}
        for idx, (name, rows, cols) in enumerate(specs):
            tseed = seed * 1_000_003 + idx
            if rows is None:
                data = (1.0 + synth.gauss(tseed, cols, sigma=0.02)).astype(np.float32)
                tensors[name] = Tensor(name, DType.F32, (cols,), data)
            else:
                dt = quant_scheme(name, scheme)
                tensors[name] = Tensor(name, dt, (cols, rows), synth.gen_quant(dt, tseed, rows, cols))
        return cls(cfg, tensors, scheme, seed)
