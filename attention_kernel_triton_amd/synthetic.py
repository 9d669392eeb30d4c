"""Seeded synthetic inputs for the benchmark configurations.

All tensors are drawn on the CPU from ``torch.Generator().manual_seed(seed)``
as fp32 N(0, 1) and rounded to fp16, in a fixed order (q, K, V / pool, then
lengths, block table, keep draws, MagicPIG K and L), and moved to ``device``
afterwards, so the same seed gives the same inputs on every machine.

Config numbering follows the benchmark list:
  0  causal GQA prefill        Q [8,64,1024,64], K/V [8,16,1024,64]
  1  var-len causal prefill    as 0, lengths [1024, U[64,1024] x 7], padding = N(0,1)*8
  2  GQA decode                q [8,64,1,64], K/V [8,16,1024,64]
  3  paged var-len decode      B=32, Hq=32, Hkv=8, D=128, page 16, len U[256,8192]
  4a sparse-token decode       q [1,32,1,128], K/V [1,8,32000,128], keep p=0.02
  4b sparse paged (+MagicPIG)  B=3, Hq=32, Hkv=8, D=256, page 16, len U[8192,32768]

The keep-mask construction mirrors the reference harness
(sparsetoken_decode_flash_attention_redundant.py:277-296): per (b, h) draw
uniform(len) and keep entries < p; the index lists themselves are produced by
the caller (on device with kept_index.select_kept, or by the oracle).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

SEED = 20240601


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(int(seed))


def _randn(g, shape, scale=1.0) -> torch.Tensor:
    t = torch.randn(shape, generator=g, dtype=torch.float32)
    if scale != 1.0:
        t.mul_(scale)
    return t.half()


@dataclass
class Prefill:
    Q: torch.Tensor
    K: torch.Tensor
    V: torch.Tensor
    causal: bool
    scale: float
    group: int
    varlen: torch.Tensor | None = None

    def to(self, device):
        return Prefill(self.Q.to(device), self.K.to(device), self.V.to(device), self.causal,
                       self.scale, self.group,
                       None if self.varlen is None else self.varlen.to(device))

    def flops(self) -> int:
        """Algorithmic FLOPs: 4*D per (query, visible key) pair."""
        B, H, S, D = self.Q.shape
        lens = [S] * B if self.varlen is None else [int(x) for x in self.varlen.tolist()]
        pairs = sum((L * (L + 1) // 2) if self.causal else L * S for L in lens)
        return 4 * D * H * pairs


def prefill_config(cfg: int = 0, seed: int = SEED, B=8, Hq=64, Hkv=16, S=1024, D=64,
                   causal=True) -> Prefill:
    g = _gen(seed + cfg)
    Q = _randn(g, (B, Hq, S, D))
    K = _randn(g, (B, Hkv, S, D))
    V = _randn(g, (B, Hkv, S, D))
    varlen = None
    if cfg == 1:
        lens = torch.randint(64, S + 1, (B,), generator=g, dtype=torch.int64)
        lens[0] = S
        varlen = lens
        # Overwrite padding rows with finite garbage that must never reach valid rows.
        for b in range(B):
            L = int(lens[b])
            if L < S:
                Q[b, :, L:] = _randn(g, (Hq, S - L, D), 8.0)
                K[b, :, L:] = _randn(g, (Hkv, S - L, D), 8.0)
                V[b, :, L:] = _randn(g, (Hkv, S - L, D), 8.0)
    return Prefill(Q, K, V, causal, 1.0 / math.sqrt(D), Hq // Hkv, varlen)


@dataclass
class Decode:
    q: torch.Tensor
    K: torch.Tensor
    V: torch.Tensor
    scale: float
    group: int

    def to(self, device):
        return Decode(self.q.to(device), self.K.to(device), self.V.to(device), self.scale, self.group)

    def bytes(self) -> int:
        return (self.K.numel() + self.V.numel() + 2 * self.q.numel()) * 2


def decode_config(seed: int = SEED, B=8, Hq=64, Hkv=16, S=1024, D=64) -> Decode:
    g = _gen(seed + 2)
    q = _randn(g, (B, Hq, 1, D))
    K = _randn(g, (B, Hkv, S, D))
    V = _randn(g, (B, Hkv, S, D))
    return Decode(q, K, V, 1.0 / math.sqrt(D), Hq // Hkv)


@dataclass
class Paged:
    q: torch.Tensor            # [B, Hq, 1, D]
    pool: torch.Tensor         # [P, 2, Hkv, page, D]
    indptr: torch.Tensor       # int32 [B+1]
    indices: torch.Tensor      # int32 [P_used]
    last_len: torch.Tensor     # int32 [B]
    lens: list = field(default_factory=list)

    def to(self, device):
        return Paged(self.q.to(device), self.pool.to(device), self.indptr.to(device),
                     self.indices.to(device), self.last_len.to(device), list(self.lens))

    def bytes(self) -> int:
        """Algorithmic HBM bytes: K and V rows of every token once, q, o and the page table."""
        Hkv, D = self.pool.shape[2], self.pool.shape[4]
        kv = sum(self.lens) * Hkv * D * 2 * 2
        qo = 2 * self.q.numel() * 2
        table = 4 * (self.indices.numel() + self.indptr.numel() + self.last_len.numel())
        return kv + qo + table


def block_table(g, lens, page: int, extra_pages: int = 0):
    """CSR page table for sequences of the given lengths over a randomly permuted pool."""
    pages = [max(1, -(-L // page)) if L > 0 else 0 for L in lens]
    last = [L - page * (n - 1) if n > 0 else 0 for L, n in zip(lens, pages)]
    total = sum(pages)
    perm = torch.randperm(total + extra_pages, generator=g)[:total].to(torch.int32)
    indptr = torch.zeros(len(lens) + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(torch.tensor(pages, dtype=torch.int64), 0).to(torch.int32)
    return indptr, perm, torch.tensor(last, dtype=torch.int32), total + extra_pages


def paged_config(seed: int = SEED, B=32, Hq=32, Hkv=8, D=128, page=16, min_len=256,
                 max_len=8192, extra_pages=0) -> Paged:
    g = _gen(seed + 3)
    q = _randn(g, (B, Hq, 1, D))
    lens = torch.randint(min_len, max_len + 1, (B,), generator=g).tolist()
    indptr, indices, last, P = block_table(g, lens, page, extra_pages)
    pool = _randn(g, (P, 2, Hkv, page, D))
    return Paged(q, pool, indptr, indices, last, lens)


@dataclass
class Sparse:
    q: torch.Tensor
    K: torch.Tensor            # dense [B, Hkv, S, D] (4a) or None
    V: torch.Tensor
    uniform: torch.Tensor      # fp32 [B, Hq, N] keep draws (entries >= row_len unused)
    row_len: torch.Tensor      # int32 [B, Hq] candidate tokens per row
    kept_ratio: float
    l_max: int
    scale: float
    group: int
    paged: Paged | None = None
    lsh_k: torch.Tensor | None = None
    lsh_l: torch.Tensor | None = None

    def to(self, device):
        mv = lambda t: None if t is None else t.to(device)  # noqa: E731
        return Sparse(mv(self.q), mv(self.K), mv(self.V), mv(self.uniform), mv(self.row_len),
                      self.kept_ratio, self.l_max, self.scale, self.group,
                      None if self.paged is None else self.paged.to(device),
                      mv(self.lsh_k), mv(self.lsh_l))


def sparse_config(seed: int = SEED, B=1, Hq=32, Hkv=8, S=32000, D=128, kept_ratio=0.02) -> Sparse:
    """Config 4a: dense cache, per-head Bernoulli keep masks over all S tokens."""
    g = _gen(seed + 4)
    q = _randn(g, (B, Hq, 1, D))
    K = _randn(g, (B, Hkv, S, D))
    V = _randn(g, (B, Hkv, S, D))
    uniform = torch.rand((B, Hq, S), generator=g, dtype=torch.float32)
    row_len = torch.full((B, Hq), S, dtype=torch.int32)
    l_max = int(S * (kept_ratio + 0.1))  # as sparsetoken_decode_flash_attention_redundant.py:278
    return Sparse(q, K, V, uniform, row_len, kept_ratio, l_max, 1.0 / math.sqrt(D), Hq // Hkv)


def sparse_paged_config(seed: int = SEED, B=3, Hq=32, Hkv=8, D=256, page=16, min_len=8192,
                        max_len=32768, kept_ratio=0.02, magicpig=True) -> Sparse:
    """Config 4b: paged var-len cache, keep masks over each sequence's tokens, MagicPIG K/L."""
    g = _gen(seed + 5)
    q = _randn(g, (B, Hq, 1, D))
    lens = torch.randint(min_len, max_len + 1, (B,), generator=g).tolist()
    indptr, indices, last, P = block_table(g, lens, page)
    pool = _randn(g, (P, 2, Hkv, page, D))
    n = max(lens)
    uniform = torch.rand((B, Hq, n), generator=g, dtype=torch.float32)
    row_len = torch.tensor(lens, dtype=torch.int32).view(B, 1).expand(B, Hq).contiguous()
    max_pages = int((indptr[1:] - indptr[:-1]).max())
    l_max = max_pages * page  # as ..._var_len_paged.py:334
    lk = ll = None
    if magicpig:
        lk = torch.rand((B, Hq), generator=g, dtype=torch.float32) * 5 + 1
        ll = torch.rand((B, Hq), generator=g, dtype=torch.float32) * 5 + 1
    paged = Paged(q, pool, indptr, indices, last, lens)
    return Sparse(q, None, None, uniform, row_len, kept_ratio, l_max, 1.0 / math.sqrt(D),
                  Hq // Hkv, paged, lk, ll)
