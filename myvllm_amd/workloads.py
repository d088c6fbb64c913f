"""Seeded synthetic inputs for the GDN path's benchmark and parity workloads.

Every tensor is drawn on the CPU from one ``torch.Generator().manual_seed(seed)``
in a fixed order, so the CPU oracle and the GPU kernels see identical bits;
callers copy to the device themselves.  Distributions follow the GDN layer's
input contract (``layers/linear_attention.py:89-90``, ``:113-114`` of
yuyifanbupt/myvllm): q, k ~ N(0, 1) then L2-normalised per head, v ~ N(0, 1),
beta = sigmoid(N(0, 1)), g = -softplus(N(0, 1)).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

HK, HV, DK, DV = 16, 32, 128, 128
CONV_DIM = 2 * HK * DK + HV * DV  # 8192 = q 2048 | k 2048 | v 4096
CONV_WIDTH = 4


def gdn_inputs(
    gen: torch.Generator,
    T: int,
    Hk: int = HK,
    Hv: int = HV,
    K: int = DK,
    V: int = DV,
    dtype: torch.dtype = torch.bfloat16,
    beta_dtype: torch.dtype = torch.float32,
    g_scale: float = 1.0,
):
    """q, k, v (rounded once to ``dtype``), g (fp32), beta, in that draw order."""
    q = F.normalize(torch.randn(T, Hk, K, generator=gen), dim=-1).to(dtype)
    k = F.normalize(torch.randn(T, Hk, K, generator=gen), dim=-1).to(dtype)
    v = torch.randn(T, Hv, V, generator=gen).to(dtype)
    g = -F.softplus(torch.randn(T, Hv, generator=gen)) * g_scale
    beta = torch.sigmoid(torch.randn(T, Hv, generator=gen)).to(beta_dtype)
    return q, k, v, g, beta


def cu_from_lengths(lengths) -> torch.Tensor:
    lens = torch.as_tensor(lengths, dtype=torch.int64)
    return torch.cat([torch.zeros(1, dtype=torch.int64), lens.cumsum(0)]).to(torch.int32)


@dataclass
class PrefillCase:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    g: torch.Tensor
    beta: torch.Tensor
    state: torch.Tensor  # (num_slots, Hv, K, V) fp32
    idx: torch.Tensor  # (N,) int32
    cu: torch.Tensor  # (N+1,) int32

    @property
    def tokens(self) -> int:
        return int(self.cu[-1])


def prefill_case(
    lengths,
    seed: int = 0,
    num_slots: int | None = None,
    Hk: int = HK,
    Hv: int = HV,
    state_std: float = 0.1,
    g_scale: float = 1.0,
    beta_dtype: torch.dtype = torch.float32,
    dtype: torch.dtype = torch.bfloat16,
    K: int = DK,
    V: int = DV,
) -> PrefillCase:
    """Chunked-prefill inputs for given sequence lengths (draws after the lengths)."""
    gen = torch.Generator().manual_seed(seed)
    N = len(lengths)
    cu = cu_from_lengths(lengths)
    T = int(cu[-1])
    q, k, v, g, beta = gdn_inputs(gen, T, Hk, Hv, K=K, V=V, dtype=dtype, beta_dtype=beta_dtype, g_scale=g_scale)
    num_slots = num_slots or max(N, 1)
    state = torch.randn(num_slots, Hv, K, V, generator=gen) * state_std
    idx = torch.randperm(num_slots, generator=gen)[:N].to(torch.int32)
    return PrefillCase(q, k, v, g, beta, state, idx, cu)


def prefill_32k_case(seed: int = 0) -> PrefillCase:
    """Chunked GDN prefill workload: 16 sequences, lengths uniform in [512, 4096]
    (seed 0: 35,846 tokens, 567 chunks of 64), Hk 16 / Hv 32, d 128, bf16 q/k/v,
    fp32 g/beta, fp32 initial state ~N(0, 0.1) in a 64-slot cache."""
    gen = torch.Generator().manual_seed(seed)
    lengths = torch.randint(512, 4097, (16,), generator=gen).tolist()
    return prefill_case(lengths, seed=seed + 1, num_slots=64)


def prefill_short_case(seed: int = 0) -> PrefillCase:
    """Many short sequences, as a chunked-prefill scheduler sends them: 512
    sequences of 64 tokens (32,768 tokens, one chunk each), Hk 16 / Hv 32,
    d 128, bf16 q/k/v, fp32 g/beta, fp32 initial state ~N(0, 0.1) in a
    512-slot cache.  Each (sequence, v-head) reads and writes its 64 KiB state
    once per 64 tokens, so the state traffic dominates."""
    return prefill_case([64] * 512, seed=seed + 5, num_slots=512)


@dataclass
class DecodeCase:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    g: torch.Tensor
    beta: torch.Tensor
    state: torch.Tensor  # (num_slots, Hv, K, V) fp32
    idx: torch.Tensor  # (B,) int32


def decode_case(B: int = 256, num_slots: int = 1024, seed: int = 0, Hk: int = HK, Hv: int = HV,
                K: int = DK, V: int = DV, dtype=torch.bfloat16, beta_dtype=torch.float32,
                state: bool = True) -> DecodeCase:
    """Recurrent decode workload: B sequences x 1 token, fp32 state cache
    (num_slots, Hv, K, V) ~N(0, 0.1), slots = randperm(num_slots)[:B].
    With ``state=False`` the cache is left for the caller to fill (used by
    the benchmark to build the 2 GiB cache on the device)."""
    gen = torch.Generator().manual_seed(seed)
    q, k, v, g, beta = gdn_inputs(gen, B, Hk, Hv, K, V, dtype=dtype, beta_dtype=beta_dtype)
    idx = torch.randperm(num_slots, generator=gen)[:B].to(torch.int32)
    st = torch.randn(num_slots, Hv, K, V, generator=gen) * 0.1 if state else None
    return DecodeCase(q, k, v, g, beta, st, idx)


@dataclass
class ConvCase:
    x: torch.Tensor
    weight: torch.Tensor
    state: torch.Tensor
    idx: torch.Tensor
    cu: torch.Tensor | None


def conv_prefill_case(lengths=None, seed: int = 0, D: int = CONV_DIM, W: int = CONV_WIDTH, num_slots: int = 1024,
                      dtype=torch.bfloat16, state_dtype=torch.float32) -> ConvCase:
    """Varlen conv workload: by default 8 sequences, lengths uniform in [256, 4096]
    (seed 0: [2943, 3503, 2192, 1807, 3696, 649, 3521, 1451], 19,762 tokens),
    8192 channels, width 4, x and w ~N(0, 0.02) bf16, no bias, fp32 conv state."""
    gen = torch.Generator().manual_seed(seed)
    if lengths is None:
        lengths = torch.randint(256, 4097, (8,), generator=gen).tolist()
    cu = cu_from_lengths(lengths)
    T = int(cu[-1])
    x = (torch.randn(T, D, generator=gen) * 0.02).to(dtype)
    w = (torch.randn(D, W, generator=gen) * 0.02).to(dtype)
    st = (torch.randn(num_slots, W - 1, D, generator=gen) * 0.02).to(dtype).to(state_dtype)
    idx = torch.randperm(num_slots, generator=gen)[: len(lengths)].to(torch.int32)
    return ConvCase(x, w, st, idx, cu)


def conv_decode_case(B: int = 256, seed: int = 0, D: int = CONV_DIM, W: int = CONV_WIDTH, num_slots: int = 1024,
                     dtype=torch.bfloat16, state_dtype=torch.float32) -> ConvCase:
    """Decode conv workload: B tokens, width-W conv state per slot (fp32), 1024 slots."""
    gen = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, D, generator=gen) * 0.02).to(dtype)
    w = (torch.randn(D, W, generator=gen) * 0.02).to(dtype)
    st = (torch.randn(num_slots, W - 1, D, generator=gen) * 0.02).to(dtype).to(state_dtype)
    idx = torch.randperm(num_slots, generator=gen)[:B].to(torch.int32)
    return ConvCase(x, w, st, idx, None)


@dataclass
class FusedDecodeCase:
    mixed_qkv: torch.Tensor  # (B, 2 Hk K + Hv V)
    conv_weight: torch.Tensor  # (D, 4)
    conv_state: torch.Tensor  # (conv_slots, 3, D)
    conv_idx: torch.Tensor  # (B,)
    a: torch.Tensor  # (B, Hv)
    b: torch.Tensor  # (B, Hv)
    A_log: torch.Tensor  # (Hv,)
    dt_bias: torch.Tensor  # (Hv,)
    state: torch.Tensor | None  # (slots, Hv, K, V) fp32
    idx: torch.Tensor  # (B,)
    Hk: int


def decode_fused_case(B: int = 256, num_slots: int = 1024, seed: int = 0, Hk: int = HK, Hv: int = HV,
                      K: int = DK, V: int = DV, dtype=torch.bfloat16, conv_state_dtype=torch.float32,
                      weight_dtype=None, state: bool = True) -> FusedDecodeCase:
    """Fused decode workload (conv update + L2 norm + gating + recurrent step):
    B sequences x 1 token of the packed q|k|v projections ~N(0, 1), conv taps
    ~N(0, 0.3), conv state ~N(0, 1), a, b ~N(0, 1) in ``dtype``,
    A_log = log U(1, 16), dt_bias = 1 (the layer's initialisation), fp32
    recurrent state ~N(0, 0.1); the conv and recurrent caches have
    ``num_slots`` slots each and are indexed by independent permutations."""
    gen = torch.Generator().manual_seed(seed)
    D = 2 * Hk * K + Hv * V
    x = torch.randn(B, D, generator=gen).to(dtype)
    w = (torch.randn(D, CONV_WIDTH, generator=gen) * 0.3).to(weight_dtype or dtype)
    cs = torch.randn(num_slots, CONV_WIDTH - 1, D, generator=gen).to(dtype).to(conv_state_dtype)
    a = torch.randn(B, Hv, generator=gen).to(dtype)
    b = torch.randn(B, Hv, generator=gen).to(dtype)
    A_log = torch.log(torch.rand(Hv, generator=gen) * 15 + 1)
    dt_bias = torch.ones(Hv)
    cidx = torch.randperm(num_slots, generator=gen)[:B].to(torch.int32)
    idx = torch.randperm(num_slots, generator=gen)[:B].to(torch.int32)
    st = torch.randn(num_slots, Hv, K, V, generator=gen) * 0.1 if state else None
    return FusedDecodeCase(x, w, cs, cidx, a, b, A_log, dt_bias, st, idx, Hk)


# ---- full-attention layers of the hybrid stack ---------------------------------------
# 16 query heads, 2 kv heads, head dim 256 (configs/qwen3_5.py:34, :93, :97).
ATTN_HQ, ATTN_HKV, ATTN_D = 16, 2, 256


@dataclass
class AttnVarlenCase:
    q: torch.Tensor  # (T, Hq, D)
    k: torch.Tensor  # (T, Hkv, D)
    v: torch.Tensor
    cu: torch.Tensor  # (N+1,) int32
    scale: float

    @property
    def max_len(self) -> int:
        return int((self.cu[1:] - self.cu[:-1]).max()) if self.cu.numel() > 1 else 0


def attn_varlen_case(lengths, seed: int = 0, Hq: int = ATTN_HQ, Hkv: int = ATTN_HKV, D: int = ATTN_D,
                     dtype=torch.bfloat16) -> AttnVarlenCase:
    """Packed q, k, v ~N(0, 1) in ``dtype`` for the given lengths; scale D^-1/2."""
    gen = torch.Generator().manual_seed(seed)
    cu = cu_from_lengths(lengths)
    T = int(cu[-1])
    q = torch.randn(T, Hq, D, generator=gen).to(dtype)
    k = torch.randn(T, Hkv, D, generator=gen).to(dtype)
    v = torch.randn(T, Hkv, D, generator=gen).to(dtype)
    return AttnVarlenCase(q, k, v, cu, D ** -0.5)


def attn_prefill_32k_case(seed: int = 0) -> AttnVarlenCase:
    """Causal varlen prefill of an attention layer over the same 16 sequence
    lengths as the GDN prefill workload (uniform in [512, 4096], seed 0)."""
    gen = torch.Generator().manual_seed(seed)
    lengths = torch.randint(512, 4097, (16,), generator=gen).tolist()
    return attn_varlen_case(lengths, seed=seed + 1)


@dataclass
class PagedCase:
    q: torch.Tensor  # (T, Hq, D): the new tokens (one per sequence for decode)
    k_cache: torch.Tensor  # (num_blocks, page, Hkv, D)
    v_cache: torch.Tensor
    block_tables: torch.Tensor  # (N, max_blocks) int32, unused entries -1
    context_lens: torch.Tensor  # (N,) int32
    cu: torch.Tensor  # (N+1,) int32 rows of q per sequence
    scale: float
    page: int

    @property
    def max_len(self) -> int:
        return int((self.cu[1:] - self.cu[:-1]).max()) if self.cu.numel() > 1 else 0


def paged_case(context_lens, new_lens, page: int = 16, seed: int = 0, Hq: int = ATTN_HQ, Hkv: int = ATTN_HKV,
               D: int = ATTN_D, dtype=torch.bfloat16, spare_blocks: int = 3) -> PagedCase:
    """A paged KV cache holding ``context_lens[n]`` keys of sequence n (the
    last ``new_lens[n]`` of which are the new tokens' own keys), pages drawn
    as a random permutation of the cache blocks; q ~N(0, 1) for the new tokens."""
    gen = torch.Generator().manual_seed(seed)
    ctx = torch.as_tensor(context_lens, dtype=torch.int64)
    new = torch.as_tensor(new_lens, dtype=torch.int64)
    npages = (ctx + page - 1) // page
    num_blocks = int(npages.sum()) + spare_blocks
    cols = max(int(npages.max()) if len(npages) else 1, 1)
    kc = torch.randn(num_blocks, page, Hkv, D, generator=gen).to(dtype)
    vc = torch.randn(num_blocks, page, Hkv, D, generator=gen).to(dtype)
    perm = torch.randperm(num_blocks, generator=gen)
    tab = torch.full((len(ctx), cols), -1, dtype=torch.int32)
    o = 0
    for n, p in enumerate(npages.tolist()):
        tab[n, :p] = perm[o:o + p].to(torch.int32)
        o += p
    cu = cu_from_lengths(new.tolist())
    q = torch.randn(int(cu[-1]), Hq, D, generator=gen).to(dtype)
    return PagedCase(q, kc, vc, tab, ctx.to(torch.int32), cu, D ** -0.5, page)


def attn_decode_case(B: int = 256, seed: int = 0, page: int = 16, lo: int = 512, hi: int = 4096,
                     **kw) -> PagedCase:
    """Paged decode of an attention layer: B sequences with context lengths
    uniform in [lo, hi], one new query each, 16-token pages."""
    gen = torch.Generator().manual_seed(seed)
    ctx = torch.randint(lo, hi + 1, (B,), generator=gen).tolist()
    return paged_case(ctx, [1] * B, page=page, seed=seed + 1, **kw)


def attn_paged_prefill_case(seed: int = 0, **kw) -> PagedCase:
    """Chunked prefill over a paged cache: 16 sequences with a cached prefix
    uniform in [0, 4096] and a new chunk uniform in [256, 2048] (whose keys are
    already in the cache), 16-token pages."""
    gen = torch.Generator().manual_seed(seed)
    new = torch.randint(256, 2049, (16,), generator=gen)
    prefix = torch.randint(0, 4097, (16,), generator=gen)
    return paged_case((prefix + new).tolist(), new.tolist(), seed=seed + 1, **kw)
