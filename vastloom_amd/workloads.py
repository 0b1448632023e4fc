"""Seeded synthetic inputs for the five benchmark and parity workloads.

No checkpoints are available offline, so every workload is generated from its seed with numpy's
PCG64. Each independent piece draws from its own stream, ``Generator(PCG64(SeedSequence([seed,
role, index])))``, so any one expert or matrix can be regenerated without the others:

  role 0  router weights, float32 N(0, 0.02), [experts, width] row-major
  role 1  expert ``index`` (the shared expert is index ``experts``): gate, then up, then down,
          each matrix drawing its block scales first and its payload bytes second
  role 2  token activations, float32 N(0, 1), [tokens, width]
  role 3  routing table draws (Zipf workload)

Block scales are binary16, rounded to nearest-even from the float32 draw. Payload bytes are
uniform: for Q8_0 the int8 quants are uniform on [-127, 127]; for IQ2_XXS, IQ3_XXS, IQ1_S and
IQ2_S every byte is uniform on [0, 255], which always decodes (every grid index, sign field and
scale field is valid); Q4_K/Q5_K/Q6_K draw their fp16 d (and dmin) scaled down by the 6-bit
sub-block scales' range, MXFP4 an E8M0 scale in [2^-10, 2^-4], BF16 truncated normal values.
Matrices are in GGUF block layout, row-major: row r's blocks are contiguous.

Workload shapes (the model shapes they mimic are OLMoE-1B-7B experts and DeepSeek-class
routed experts):

  q8_expert      Q8_0 expert, width 2048, expert width 1024, one token                    seed 0
  q8_moe         64 Q8_0 experts as above, softmax router, top-8 renormalised, one token     seed 1
  iq2_moe        256 IQ2_XXS experts + 1 shared, width 7168, expert width 2048, sigmoid
                 router, top-8, one token                                                    seed 2
  mixed_moe      as iq2_moe with IQ1_S gate/up and IQ3_XXS down, five tokens                 seed 3
  grouped_moe    as iq2_moe, 512 tokens, table routing drawn from Zipf(1.1) over experts     seed 4
  kquant_moe     as iq2_moe with Q4_K gate/up and Q6_K down (GGUF-layout types), one token   seed 5
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

F32, Q8_0, IQ2_XXS, IQ3_XXS, IQ1_S = 0, 8, 16, 18, 19
Q4_K, Q5_K, Q6_K, IQ2_S, BF16, MXFP4 = 12, 13, 14, 22, 30, 39

# (block elements, block bytes) of each GGUF storage type (ggml_quantization.hpp:13-28).
BLOCK = {F32: (1, 4), Q8_0: (32, 34), IQ2_XXS: (256, 66), IQ3_XXS: (256, 98), IQ1_S: (256, 50),
         Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), IQ2_S: (256, 82), BF16: (1, 2),
         MXFP4: (32, 17)}
TYPE_NAMES = {F32: "f32", Q8_0: "q8_0", IQ2_XXS: "iq2_xxs", IQ3_XXS: "iq3_xxs", IQ1_S: "iq1_s",
              Q4_K: "q4_k", Q5_K: "q5_k", Q6_K: "q6_k", IQ2_S: "iq2_s", BF16: "bf16",
              MXFP4: "mxfp4"}


def storage_bytes(qtype: int, rows: int, cols: int) -> int:
    be, bb = BLOCK[qtype]
    if cols % be:
        raise ValueError(f"{TYPE_NAMES[qtype]} needs columns divisible by {be}, got {cols}")
    return rows * (cols // be) * bb


def _rng(seed: int, role: int, index: int = 0) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, role, index])))


def _fp16_scales(rng: np.random.Generator, n: int, factor: float) -> np.ndarray:
    d = (np.abs(rng.standard_normal(n)) * factor).astype(np.float32)
    return d.astype(np.float16).view(np.uint16)


def random_matrix(rng: np.random.Generator, qtype: int, rows: int, cols: int,
                  scale_factor: float) -> np.ndarray:
    """One matrix in GGUF block layout as a flat uint8 array."""
    be, bb = BLOCK[qtype]
    if qtype == F32:
        return rng.standard_normal(rows * cols).astype(np.float32).view(np.uint8)
    if qtype == BF16:  # N(0, scale_factor) truncated to its upper 16 bits
        v = (rng.standard_normal(rows * cols) * scale_factor).astype(np.float32)
        return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
    blocks = rows * (cols // be)
    if qtype == MXFP4:  # E8M0 scales 2^-10 .. 2^-4, uniform code bytes
        out = rng.integers(0, 256, size=(blocks, bb), dtype=np.uint8)
        out[:, 0] = rng.integers(118, 125, size=blocks, dtype=np.uint8)
        return out.reshape(-1)
    if qtype == Q6_K:  # fp16 d at byte 208; quants and int8 sub-block scales uniform
        scales = _fp16_scales(rng, blocks, scale_factor / 32.0)
        out = rng.integers(0, 256, size=(blocks, bb), dtype=np.uint8)
        out[:, 208] = scales & 0xFF
        out[:, 209] = scales >> 8
        return out.reshape(-1)
    if qtype in (Q4_K, Q5_K):  # fp16 d and dmin, then uniform scale and quant bytes
        scales = _fp16_scales(rng, 2 * blocks, scale_factor / 16.0).reshape(blocks, 2)
        out = rng.integers(0, 256, size=(blocks, bb), dtype=np.uint8)
        out[:, 0], out[:, 1] = scales[:, 0] & 0xFF, scales[:, 0] >> 8
        out[:, 2], out[:, 3] = scales[:, 1] & 0xFF, scales[:, 1] >> 8
        return out.reshape(-1)
    scales = _fp16_scales(rng, blocks, scale_factor)
    out = np.empty((blocks, bb), np.uint8)
    out[:, 0] = scales & 0xFF
    out[:, 1] = scales >> 8
    if qtype == Q8_0:
        out[:, 2:] = rng.integers(-127, 128, size=(blocks, bb - 2), dtype=np.int16).astype(
            np.int8).view(np.uint8)
    else:
        out[:, 2:] = rng.integers(0, 256, size=(blocks, bb - 2), dtype=np.uint8)
    return out.reshape(-1)


@dataclass
class Expert:
    gate: np.ndarray
    up: np.ndarray
    down: np.ndarray
    gate_type: int
    down_type: int

    def triple(self):
        return ((self.gate_type, self.gate), (self.gate_type, self.up),
                (self.down_type, self.down))


@dataclass
class MoeWorkload:
    name: str
    seed: int
    width: int
    intermediate: int
    experts: int
    top_k: int
    tokens: int
    gate_type: int
    down_type: int
    scale_factor: float
    semantics: str            # "qwen" (softmax, post-down weight) or "deepseek"
    score_fn: int = 1         # deepseek scoring: 0 sqrt_softplus, 1 sigmoid
    has_shared: bool = False
    routing: str = "learned"  # "learned" | "softmax" | "zipf_table"
    route_scale: float = 1.0
    swiglu_limit: float = 0.0
    zipf_s: float = 1.1
    _cache: dict = field(default_factory=dict, repr=False)

    # -- generated pieces ------------------------------------------------------------
    def router(self) -> np.ndarray:
        if "router" not in self._cache:
            r = _rng(self.seed, 0).standard_normal(self.experts * self.width)
            self._cache["router"] = (r * 0.02).astype(np.float32).reshape(self.experts,
                                                                          self.width)
        return self._cache["router"]

    def expert(self, index: int) -> Expert:
        """Expert ``index``; index == experts is the shared expert."""
        rng = _rng(self.seed, 1, index)
        H, F = self.width, self.intermediate
        gate = random_matrix(rng, self.gate_type, F, H, self.scale_factor)
        up = random_matrix(rng, self.gate_type, F, H, self.scale_factor)
        down = random_matrix(rng, self.down_type, H, F, self.scale_factor)
        return Expert(gate, up, down, self.gate_type, self.down_type)

    def shared(self) -> Expert | None:
        return self.expert(self.experts) if self.has_shared else None

    def x(self) -> np.ndarray:
        if "x" not in self._cache:
            v = _rng(self.seed, 2).standard_normal(self.tokens * self.width)
            self._cache["x"] = v.astype(np.float32).reshape(self.tokens, self.width)
        return self._cache["x"]

    def zipf_table(self) -> np.ndarray:
        """Per-token expert ids for table routing: top_k distinct ids drawn with probability
        proportional to rank^-s over a seeded permutation of the experts."""
        if "table" not in self._cache:
            rng = _rng(self.seed, 3)
            perm = rng.permutation(self.experts)
            p = np.arange(1, self.experts + 1, dtype=np.float64) ** (-self.zipf_s)
            p /= p.sum()
            table = np.empty((self.tokens, self.top_k), np.uint32)
            for t in range(self.tokens):
                table[t] = perm[rng.choice(self.experts, self.top_k, replace=False, p=p)]
            self._cache["table"] = table
        return self._cache["table"]

    @property
    def model(self) -> str:
        """The model family whose shapes the workload mimics."""
        return "OLMoE-1B-7B-shaped" if self.width == 2048 else "DeepSeek-class"

    @property
    def kind(self) -> str:
        return "single-expert SwiGLU FFN" if self.routing == "single" else "MoE layer"

    # -- byte accounting ---------------------------------------------------------------
    def expert_bytes(self) -> int:
        H, F = self.width, self.intermediate
        return 2 * storage_bytes(self.gate_type, F, H) + storage_bytes(self.down_type, H, F)

    def router_bytes(self) -> int:
        return self.experts * self.width * 4


def workload(name: str) -> MoeWorkload:
    if name == "q8_expert":
        return MoeWorkload(name, 0, 2048, 1024, 1, 1, 1, Q8_0, Q8_0, 0.002, "qwen",
                           routing="single")
    if name == "q8_moe":
        return MoeWorkload(name, 1, 2048, 1024, 64, 8, 1, Q8_0, Q8_0, 0.002, "qwen",
                           routing="softmax")
    if name == "iq2_moe":
        return MoeWorkload(name, 2, 7168, 2048, 256, 8, 1, IQ2_XXS, IQ2_XXS, 0.01, "deepseek",
                           score_fn=1, has_shared=True)
    if name == "mixed_moe":
        return MoeWorkload(name, 3, 7168, 2048, 256, 8, 5, IQ1_S, IQ3_XXS, 0.01, "deepseek",
                           score_fn=1, has_shared=True)
    if name == "kquant_moe":
        return MoeWorkload(name, 5, 7168, 2048, 256, 8, 1, Q4_K, Q6_K, 0.01, "deepseek",
                           score_fn=1, has_shared=True)
    if name == "grouped_moe":
        return MoeWorkload(name, 4, 7168, 2048, 256, 8, 512, IQ2_XXS, IQ2_XXS, 0.01,
                           "deepseek", score_fn=1, has_shared=True, routing="zipf_table")
    raise KeyError(name)


WORKLOADS = ("q8_expert", "q8_moe", "iq2_moe", "mixed_moe", "grouped_moe", "kquant_moe")
