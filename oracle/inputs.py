"""Deterministic synthetic inputs for the ring-attention path (TEST INFRASTRUCTURE).

This module belongs to the oracle: only tests, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product path never does.

Generator
---------
A 64-bit LCG followed by Box-Muller, as the reference's pure-Rust correctness model
defines it (``rust/src/smoke/reference_algo.rs:56-90``):

* ``state = state * 6364136223846793005 + 1442695040888963407  (mod 2**64)``
* ``u = ((state >> 11) + 0.5) / 2**53``                      (open interval (0, 1))
* ``r = sqrt(-2 ln u1)``, ``theta = 2 pi u2``; the first draw of a pair returns
  ``r cos theta`` and keeps ``r sin theta`` as the spare for the next draw.

Q, then K, then V are drawn from ONE stream, in that order
(``rust/src/smoke/correctness.rs:11-29``), each tensor in token-major order
``[seq, heads, dim]`` (the ``Tensor3`` layout, ``reference_algo.rs:7-45``).  The seed
of config ``i`` (0-based) is ``42 + i`` (``rust/src/lib.rs:109-118``).  Values are
f64, then rounded to fp32, then (for bf16 configs) to bf16 by round-to-nearest-even.

The LCG is evaluated with exact jump-ahead so that hundreds of millions of draws take
seconds: after ``n`` steps ``s_n = A_n s_0 + C_n`` with ``A_n = a**n`` and
``C_n = c (1 + a + ... + a**(n-1))``, all mod 2**64 (numpy uint64 arithmetic wraps).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

LCG_A = 6364136223846793005
LCG_C = 1442695040888963407
_MASK = (1 << 64) - 1
_BLOCK = 1 << 16


def lcg_scalar_states(seed: int, n: int) -> list[int]:
    """Pure-Python LCG (the recurrence exactly as written); used to pin the vector path."""
    s = seed & _MASK
    out = []
    for _ in range(n):
        s = (s * LCG_A + LCG_C) & _MASK
        out.append(s)
    return out


def _jump_tables(n: int) -> tuple[np.ndarray, np.ndarray]:
    """A[k] = a**(k+1), C[k] = c*(1+...+a**k) (mod 2**64) for k < n, computed exactly."""
    a_tab = np.empty(n, dtype=np.uint64)
    c_tab = np.empty(n, dtype=np.uint64)
    a_pow, c_acc = 1, 0
    # Build in Python ints for exactness, in chunks to keep it quick.
    for k in range(n):
        c_acc = (c_acc * LCG_A + LCG_C) & _MASK  # value after k+1 steps from state 0
        a_pow = (a_pow * LCG_A) & _MASK
        a_tab[k] = a_pow
        c_tab[k] = c_acc
    return a_tab, c_tab


_TABLES: dict[int, tuple[np.ndarray, np.ndarray]] = {}


def _tables(n: int) -> tuple[np.ndarray, np.ndarray]:
    if n not in _TABLES:
        _TABLES[n] = _jump_tables(n)
    return _TABLES[n]


def lcg_states(seed: int, n: int, block: int = _BLOCK) -> np.ndarray:
    """States s_1..s_n of the LCG started at ``seed`` (vectorised jump-ahead)."""
    out = np.empty(n, dtype=np.uint64)
    blk = min(block, max(n, 1))
    a_tab, c_tab = _tables(blk)
    s = np.uint64(seed & _MASK)
    pos = 0
    with np.errstate(over="ignore"):
        while pos < n:
            m = min(blk, n - pos)
            seg = a_tab[:m] * s + c_tab[:m]
            out[pos:pos + m] = seg
            s = seg[-1]
            pos += m
    return out


def uniforms_open01(states: np.ndarray) -> np.ndarray:
    """``((state >> 11) + 0.5) / 2**53`` as f64 (reference_algo.rs:66-74)."""
    return ((states >> np.uint64(11)).astype(np.float64) + 0.5) / float(1 << 53)


class NormalStream:
    """Stateful standard-normal stream with the reference's spare semantics."""

    def __init__(self, seed: int):
        self.state = seed & _MASK
        self.spare: float | None = None

    def _advance_states(self, n: int) -> np.ndarray:
        st = lcg_states(self.state, n)
        if n:
            self.state = int(st[-1])
        return st

    def draw(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float64)
        i = 0
        if n and self.spare is not None:
            out[0] = self.spare
            self.spare = None
            i = 1
        rem = n - i
        pairs = (rem + 1) // 2
        if pairs:
            u = uniforms_open01(self._advance_states(2 * pairs))
            u1, u2 = u[0::2], u[1::2]
            r = np.sqrt(-2.0 * np.log(u1))
            th = 2.0 * math.pi * u2
            z = np.empty(2 * pairs, dtype=np.float64)
            z[0::2] = r * np.cos(th)
            z[1::2] = r * np.sin(th)
            out[i:] = z[:rem]
            if rem % 2 == 1:
                self.spare = float(z[-1])
        return out

    def uniform(self) -> float:
        """One ``next_f64_open01`` draw (reference_algo.rs:66-74)."""
        return float(uniforms_open01(self._advance_states(1))[0])


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit pattern (uint16), round-to-nearest-even (finite inputs)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))
    return (rounded >> np.uint32(16)).astype(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


@dataclass
class RingCase:
    """One ring-prefill configuration (BASELINE.json ``configs``)."""

    name: str
    chunks: list[int]
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    dtype: str  # "fp32" | "bf16"
    seed: int
    causal: bool = True
    extra: dict = field(default_factory=dict)

    @property
    def seq_len(self) -> int:
        return int(sum(self.chunks))

    @property
    def offsets(self) -> list[int]:
        off, out = 0, []
        for c in self.chunks:
            out.append(off)
            off += c
        return out

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.head_dim)

    def causal_flops(self) -> float:
        """Algorithmic FLOPs counting causal pairs only: 2 GEMMs x 2 x D x Hq x S(S+1)/2."""
        s = self.seq_len
        return 2.0 * self.head_dim * self.num_q_heads * s * (s + 1)


def c5_chunks(seed: int = 42, n: int = 8, total: int = 131072, unit: int = 1024,
              minimum: int = 8192) -> list[int]:
    """Seeded uneven split for the 128k staged config.

    ``n`` uniform weights from the LCG (seed 42, its own stream) share the
    ``(total - n*minimum)/unit`` spare units by largest remainder (ties to the lower
    index), added to ``n*minimum``.  Same largest-remainder idea as the reference's
    capacity split (``rust/src/capacity.rs:67-110``).
    """
    ns = NormalStream(seed)
    w = [ns.uniform() for _ in range(n)]
    spare = (total - n * minimum) // unit
    tot = sum(w)
    quota = [spare * wi / tot for wi in w]
    base = [int(math.floor(x)) for x in quota]
    left = spare - sum(base)
    order = sorted(range(n), key=lambda i: (-(quota[i] - base[i]), i))
    for i in order[:left]:
        base[i] += 1
    return [minimum + b * unit for b in base]


def config_cases() -> list[RingCase]:
    """The five BASELINE.json configs, as ring cases (c4 is decode; its fields describe it)."""
    return [
        RingCase("c1_cpu_smoke", [640, 384], 8, 8, 64, "fp32", 42),
        RingCase("c2_qwen25_3b", [4096, 2560, 1536], 16, 2, 128, "bf16", 43),
        RingCase("c3_llama3_8b", [12288, 8192, 8192, 4096], 32, 8, 128, "bf16", 44),
        RingCase("c4_paged_decode", [8192, 5120, 3072], 32, 8, 128, "bf16", 45,
                 causal=False, extra={"batch": 64, "block_size": 16, "pool_blocks": 65536}),
        RingCase("c5_staged_128k", c5_chunks(), 32, 8, 128, "bf16", 46,
                 extra={"block_size": 16}),
    ]


def make_qkv(case: RingCase, seq_len: int | None = None):
    """Draw Q [S,Hq,D], K [S,Hkv,D], V [S,Hkv,D] for ``case`` from one stream.

    Returns (q, k, v) as numpy arrays: float32 for fp32 cases, uint16 bf16 bit
    patterns for bf16 cases.  Uses the oracle's C generator (``hcp_oracle.c``), which
    :class:`NormalStream` pins on small sizes.
    """
    from . import clib

    s = case.seq_len if seq_len is None else seq_len
    shapes = [(s, case.num_q_heads, case.head_dim),
              (s, case.num_kv_heads, case.head_dim),
              (s, case.num_kv_heads, case.head_dim)]
    return tuple(clib.draw_normals(case.seed, shapes, "bf16" if case.dtype == "bf16" else "fp32"))


def to_f32(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(x) if x.dtype == np.uint16 else x.astype(np.float32)


def permuted_block_table(seed: int, num_blocks: int) -> np.ndarray:
    """Seeded Fisher-Yates permutation of ``range(num_blocks)`` (int32).

    ``for i = n-1 .. 1: j = floor(u * (i+1)); swap(p[i], p[j])`` with ``u`` the LCG's
    open-interval uniforms, one draw per step, in that order.
    """
    from . import clib

    u = clib.draw_uniforms(seed, max(num_blocks - 1, 0))
    p = np.arange(num_blocks, dtype=np.int64)
    for step, i in enumerate(range(num_blocks - 1, 0, -1)):
        j = int(u[step] * (i + 1))
        p[i], p[j] = p[j], p[i]
    return p.astype(np.int32)
