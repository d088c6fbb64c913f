// Chunked gated-delta-rule prefill, fused into one kernel per (sequence, v-head).
//
// Replaces the six-kernel Triton pipeline of chunk_gated_delta_rule
// (ops/gated_delta_rule/gated_delta_rule.py:31-66 in yuyifanbupt/myvllm:
// cumsum.py, chunk_scaled_dot_kkt.py, solve_tril.py, wu.py, h.py, o.py), which
// round-trips A, w, u, the per-chunk states h and v_new through HBM.  Here one
// 512-thread workgroup walks the chunks of one sequence for one v-head and
// keeps everything on chip; only q/k/v/g/beta are read and o written.
//
// The workgroup is split by role, and the two roles are software-pipelined
// over chunks through double-buffered LDS chunk tiles:
//  * state waves 0..3 hold the fp32 128x128 state in registers (wave w owns
//    value columns [32w, 32w+32)) and run the state products of chunk c;
//  * producer waves 4..7 stage the next chunks (K, Q, V, decays) and compute
//    everything that does not depend on the state: the kk^T and qk^T tiles,
//    T = (I + A)^-1 and P.  Waves 4 and 5 each solve one 32x32
//    diagonal block of T two chunks ahead, wave 6 stages K and the decays
//    and forms A_10 and the off-diagonal block T_10 = -T_11 A_10 T_00,
//    wave 7 stages Q, forms the three P tiles and stages V.
// Both roles execute one workgroup barrier per chunk; within a chunk the
// waves hand work to each other through LDS arrival counters.
//
// Per chunk of L <= 64 tokens (gamma = in-chunk cumsum of g):
//   A  = strict_lower(beta_i k_i.k_j e^(gamma_i - gamma_j))    (kk^T, MFMA)
//   P  = lower(q_i.k_j e^(gamma_i - gamma_j))                  (qk^T, MFMA)
//   T  = (I + A)^-1              (16x16 diagonal blocks by substitution,
//                                   off-diagonal blocks by MFMA block merges)
//   R  = diag(beta) (V - diag(e^gamma) K S)
//   V' = T R                      (= u - w S of the reference)
//   O  = scale [diag(e^gamma) Q S + P V']
//   S  = e^gamma_L S + K^T diag(e^(gamma_L - gamma)) V'
//
// The MFMAs run in fp16 (same rate as bf16).  q and k are bf16 or fp16
// values; fp16 holds a bf16 value exactly when |x| >= 2^-14 (its normal
// range) and rounds smaller components to its subnormal grid (absolute error
// <= 2^-25, nothing next to a row of norm ~1).  Every fp32 operand that feeds
// the carried state (S, R, the decayed V', T, A_10 and the merge product) is
// split into fp16 hi + lo parts (22 mantissa bits; lo x lo is dropped).  R
// and V' are first scaled by a power of two per value column (max |x| in
// [2^9, 2^10)) so fp16 can neither overflow nor flush them; the scale is
// undone on the fp32 accumulator.  The state is held in power-of-two units
// per value column that keep |S| < 2^14, so it is split as it stands.  The
// T blocks (unit diagonal) and A_10 are split unscaled.  Products that only
// feed o use the hi part.
//
// MFMA operand layouts (lane l, n = l % 32, g = l / 32), 32x32x16:
// A[m][k] lane holds row n, 8 k; B[k][n] lane holds column n, 8 k; C lane
// holds column n, rows 8i + 4g + r (i, r < 4).  A C-layout tile whose rows
// are the contraction index is fed back as a B operand without data movement
// by ordering each 16-wide k-step as k = 16s + 8*(m / 4) + 4g + (m % 4)
// (m = operand slot), and every A operand is read from LDS in that order.
// 16x16x16: A lane holds row l%16, k = 4(l/16)..+3; B column l%16, same k;
// C column l%16, rows 4(l/16)..+3 (already in B order).
#include "gdn_common.h"

namespace {

constexpr int kThreads = 512;        // 4 state waves + 4 producer waves
constexpr int C = 64;      // chunk
constexpr int KD = 128;    // key head dim
constexpr int VD = 128;    // value head dim
constexpr int LDK = 136;   // fp16 row stride of the K/Q tiles
constexpr int LDV = 144;   // bf16 row stride of the V tile (conflict-free transposed reads)
constexpr int LDH = 68;    // fp16 row stride of T_hi/T_lo/P
constexpr int kMaxRankedSeqs = 256;  // longest-first ordering for up to this many sequences

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct PrefillArgs {
  const bf16_t* q; const bf16_t* k; const bf16_t* v; const float* g; const void* beta;
  float* state; const void* idx; const void* cu; bf16_t* out;
  int64_t q_s0, q_s1, k_s0, k_s1, v_s0, v_s1, g_s0, g_s1, b_s0, b_s1, o_s0, o_s1;
  int64_t st_slot, st_head;
  int64_t T, nseq, num_slots;
  int32_t Hv, r;
  int32_t b_dtype;
  float scale;
  int32_t spin_limit;  // bound of a producer wait (sleep iterations)
  int32_t per_wg;      // 0: one item per workgroup, longest first; > 0: runs of work ids dealt by cost
  int32_t kd, vd;      // key and value head dims (multiples of 8 up to 128; smaller ones run zero-padded)
  int32_t flags;       // GDN_PREFILL_ZERO_INIT | GDN_PREFILL_ACCUM_STATE | GDN_PREFILL_ACCUM_OUT
  bool idx64, cu64;
};

// On-chip data.  The state waves work on chunk c while the producers stage
// chunk c + 1 and solve the diagonal blocks of T for chunk c + 2:
//  * per-chunk tiles, double-buffered by chunk parity (44,816 bytes each);
//  * T of three consecutive chunks, rotating (17,408 bytes each);
//  * one V tile: the state waves signal when they have read chunk c's
//    values, and only then is chunk c + 1's written.
struct ChunkTiles {
  f16_t k[C * LDK];
  f16_t q[C * LDK];  // chunk queries (the output is staged in the V tile)
  f16_t p[C * LDH];  // P (fp16), lower triangle
  alignas(16) float gam[C];
  alignas(16) float eg[C];    // e^gamma
  alignas(16) float ieg[C];   // e^-gamma
  alignas(16) float edec[C];  // e^(gamma_L - gamma), 0 past the chunk's last token
  alignas(16) float beta[C];
  float gam_last;
  int32_t fact;  // every |gamma| < 80: e^(gamma_i - gamma_j) = e^gamma_i e^-gamma_j (both normal)
};

// T = (I + A)^-1 as fp16 hi + lo.  Block (0,1) (rows 0..31,
// columns 32..63) is zero and never read by the state waves; the producers
// keep A_10 there, and while the diagonal blocks are being solved the two
// off-diagonal blocks hold the fp32 working copies of the diagonal blocks.
struct TBuf {
  f16_t hi[C * LDH];
  f16_t lo[C * LDH];
};

struct Smem {
  ChunkTiles tiles[2];
  TBuf tb[3];
  bf16_t v[C * LDV];
  alignas(16) float dvec[2][4][C];  // waves 4, 5: gamma, beta, e^gamma, e^-gamma of the chunk they solve
  float kn2[3][2];   // max_t |k_t|^2 over each diagonal block's rows, per T buffer
  int32_t kv_ready;  // chunks whose K tile and decay vectors are staged (wave 6 -> 7)
  int32_t v_free;    // state-wave arrivals after reading the V tile (4 per chunk)
  int32_t pro;       // producer arrivals at the prologue barrier
  int32_t failed;    // a producer wait gave up (a pipeline logic error): the item's output is NaN
  int32_t seq;
};
static_assert(sizeof(ChunkTiles) == 44816 && sizeof(TBuf) == 17408, "tile sizes as documented above");
static_assert(sizeof(Smem) <= 160 * 1024, "one workgroup's LDS");

GDN_DEVICE f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
GDN_DEVICE f32x4 mfma16(f16x4 a, f16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

GDN_DEVICE f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int j = 0; j < 16; ++j) z[j] = 0.f;
  return z;
}

GDN_DEVICE f16x8 cat4(f16x4 lo, f16x4 hi) {
  return (f16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Fragment of a row-major fp16 LDS matrix M: lane holds M[r0 + n][k-step
// slots] -- an A operand (rows of M are the M dim) or a B operand of M^T.
GDN_DEVICE f16x8 frag_rows(const f16_t* M, int ld, int r0, int kbase, int lane) {
  const f16_t* p = M + (r0 + (lane & 31)) * ld + kbase + 4 * (lane >> 5);
  return cat4(*reinterpret_cast<const f16x4*>(p), *reinterpret_cast<const f16x4*>(p + 8));
}

// Transposed read of a row-major 16-bit LDS matrix (ds_read_b64_tr_b16: each
// 16-lane group reads a 4x16 block, lane i gets column i).
GDN_DEVICE s16x4 tr_read(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
}
// Fragment of the transpose of a row-major fp16 LDS matrix M: lane holds
// M[k-step slots][c0 + n].
GDN_DEVICE f16x8 frag_cols(const f16_t* M, int ld, int c0, int kbase, int lane) {
  const int j = lane & 15, qd = lane >> 4;
  const f16_t* p = M + (kbase + 4 * (qd >> 1) + (j >> 2)) * ld + c0 + 16 * (qd & 1) + 4 * (j & 3);
  return cat4(__builtin_bit_cast(f16x4, tr_read(p)), __builtin_bit_cast(f16x4, tr_read(p + 8 * ld)));
}

// K and Q tiles are stored with the middle two 4-element quads of every
// 16-column group swapped (logical quad q at stored quad kq_quad(q)), so that
// the 8 k-values a lane takes for one 16-wide k-step (logical columns 4g..4g+3
// and 8+4g..8+4g+3) are 16 contiguous bytes: one ds_read_b128 per fragment
// instead of two ds_read_b64 (a wave issues one LDS read per ~35 cycles
// whatever its width, so the count of reads is what costs).  A Gram of two
// such tiles needs nothing else; the transposed reads of K (K^T as an A
// operand, whose rows are K's columns) permute their quad addresses so the
// lanes still receive logical columns in order.
GDN_DEVICE int kq_quad(int q) { return ((q & 1) << 1) | (q >> 1); }
GDN_DEVICE f16x8 frag_rows_kq(const f16_t* M, int r0, int kbase, int lane) {
  return *reinterpret_cast<const f16x8*>(M + (r0 + (lane & 31)) * LDK + kbase + 8 * (lane >> 5));
}
GDN_DEVICE f16x8 frag_cols_kq(const f16_t* M, int c0, int kbase, int lane) {
  const int j = lane & 15, qd = lane >> 4;
  const f16_t* p = M + (kbase + 4 * (qd >> 1) + (j >> 2)) * LDK + c0 + 16 * (qd & 1) + 4 * kq_quad(j & 3);
  return cat4(__builtin_bit_cast(f16x4, tr_read(p)), __builtin_bit_cast(f16x4, tr_read(p + 8 * LDK)));
}

// Per-row vector entries for C-layout rows r0 + 8i + 4g + (0..3).
GDN_DEVICE f32x4 rows4(const float* vec, int r0, int i, int lane) {
  return *reinterpret_cast<const f32x4*>(vec + r0 + 8 * i + 4 * (lane >> 5));
}

// Maximum of |x| over one value column of the wave's `nt` C tiles.  In the
// C layout lanes l and l ^ 32 hold the two row halves of column l % 32, so
// the per-lane maximum (a tree of a few dependent operations) needs one
// exchange between the wave halves; no wave-wide reduction.  Non-negative
// floats order like their bit patterns, so the exchange takes the maximum on
// integers.
GDN_DEVICE float col_max(const f32x16* t, int nt) {
  float m[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    m[j] = fabsf(t[0][j]);
    for (int i = 1; i < nt; ++i) m[j] = fmaxf(m[j], fabsf(t[i][j]));
  }
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
    for (int j = 0; j < w; ++j) m[j] = fmaxf(m[j], m[j + w]);
  const uint32_t v = __builtin_bit_cast(uint32_t, m[0]);
  const auto sw = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __builtin_bit_cast(float, max(sw[0], sw[1]));
}

// Exponent E with max|x| in [2^(E-1), 2^E) over one value column, kNone
// when the column is zero.
constexpr int kNone = -4096;
GDN_DEVICE int col_max_exp(const f32x16* t, int nt) {
  const float mx = col_max(t, nt);
  return mx > 0.f ? __builtin_amdgcn_frexp_expf(mx) : kNone;
}

// Power-of-two exponent e with max|x| * 2^-e in [2^9, 2^10) over one value
// column (0 when the column is zero).
GDN_DEVICE int col_scale_exp(const f32x16* t, int nt) {
  const int e = col_max_exp(t, nt);
  return e == kNone ? 0 : e - 10;
}

// Inclusive prefix sum over the 64 lanes (DPP row shifts, then the row
// broadcasts of the last lane of each row).
GDN_DEVICE float wave_inclusive_scan(float x) {
  x += __builtin_amdgcn_update_dpp(0.f, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0.f, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0.f, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0.f, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0.f, x, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
  x += __builtin_amdgcn_update_dpp(0.f, x, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
  return x;
}

// Maximum over the 64 lanes of a non-negative float (bit patterns order like the values).
GDN_DEVICE float wave_max(float x) {
  int v = __builtin_bit_cast(int, x);
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false));  // row_shr:1
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false));  // row_shr:2
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false));  // row_shr:4
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false));  // row_shr:8
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false));  // row_bcast:15
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false));  // row_bcast:31
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(v, 63));
}

// hi/lo fp16 splits: hi = fp16(x) (round to nearest even), lo = fp16(x - hi).
// hi is converted once and its bits are pinned through an empty asm, so the
// x - hi below is taken from exactly the bits that are stored as hi.  (If the
// compiler is left to convert x twice it may pick the packed and the scalar
// float->fp16 instructions for the two uses, and those can disagree on exact
// rounding ties, which leaves lo referenced to a different hi.)
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
GDN_DEVICE void split_pair(float x0, float x1, f16_t& h0, f16_t& h1, f16_t& l0, f16_t& l1) {
  const f32x2 x = {x0, x1};
  uint32_t hb = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, f16x2));
  asm volatile("" : "+v"(hb));
  const f16x2 h = __builtin_bit_cast(f16x2, hb);
  const f32x2 r = {x0 - (float)h[0], x1 - (float)h[1]};
  const f16x2 l = __builtin_convertvector(r, f16x2);
  h0 = h[0];
  h1 = h[1];
  l0 = l[0];
  l1 = l[1];
}

// Scaled fp16 hi/lo pairs: hi = fp16(x s) and lo = fp16(x s - hi) (s a
// power of two times a per-element factor, so x s - hi is exact in fp32 and
// each half is rounded once).  hi's bits are pinned through an empty asm, so
// lo is referenced to exactly the stored hi bits whichever conversion
// instructions the compiler picks for the two uses.  (Plain code rather than
// hand-written v_fma_mix* instructions: the compiler pads an MFMA's operand
// reads after VALU writes only for instructions it generated itself.)  A
// scale per element lets a per-row factor ride along (C-layout neighbours
// are adjacent rows).
GDN_DEVICE uint32_t mix_hi_pair(float x0, float s0, float x1, float s1) {
  const f16x2 h = {(f16_t)(x0 * s0), (f16_t)(x1 * s1)};
  uint32_t hb = __builtin_bit_cast(uint32_t, h);
  asm volatile("" : "+v"(hb));
  return hb;
}
GDN_DEVICE uint32_t mix_lo_pair(float x0, float s0, float x1, float s1, uint32_t hb) {
  const f16x2 h = __builtin_bit_cast(f16x2, hb);
  const f16x2 l = {(f16_t)__builtin_fmaf(x0, s0, -(float)h[0]), (f16_t)__builtin_fmaf(x1, s1, -(float)h[1])};
  return __builtin_bit_cast(uint32_t, l);
}

// split of registers 8h..8h+7 of a C tile, times sc
GDN_DEVICE void split8(const f32x16& c, int h, float sc, f16x8& hi, f16x8& lo) {
  uint32_t H[4], L[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    H[m] = mix_hi_pair(c[8 * h + 2 * m], sc, c[8 * h + 2 * m + 1], sc);
    L[m] = mix_lo_pair(c[8 * h + 2 * m], sc, c[8 * h + 2 * m + 1], sc, H[m]);
  }
  hi = __builtin_bit_cast(f16x8, (u32x4){H[0], H[1], H[2], H[3]});
  lo = __builtin_bit_cast(f16x8, (u32x4){L[0], L[1], L[2], L[3]});
}
// the same unscaled: hi = fp16(x), lo = fp16(fma(x, one, -hi)) with one = 1
// held opaque by the caller (the compiler would otherwise fold the fma into a
// subtraction and convert hi back to fp32 first)
GDN_DEVICE void split8u(const f32x16& c, int h, float one, f16x8& hi, f16x8& lo) {
  uint32_t H[4], L[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const f16x2 hv = {(f16_t)c[8 * h + 2 * m], (f16_t)c[8 * h + 2 * m + 1]};
    H[m] = __builtin_bit_cast(uint32_t, hv);
    asm volatile("" : "+v"(H[m]));
    L[m] = mix_lo_pair(c[8 * h + 2 * m], one, c[8 * h + 2 * m + 1], one, H[m]);
  }
  hi = __builtin_bit_cast(f16x8, (u32x4){H[0], H[1], H[2], H[3]});
  lo = __builtin_bit_cast(f16x8, (u32x4){L[0], L[1], L[2], L[3]});
}
// the same with one factor per register (f[m] scales register 8h + m)
GDN_DEVICE void split8f(const f32x16& c, int h, const float (&f)[8], f16x8& hi, f16x8& lo) {
  uint32_t H[4], L[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    H[m] = mix_hi_pair(c[8 * h + 2 * m], f[2 * m], c[8 * h + 2 * m + 1], f[2 * m + 1]);
    L[m] = mix_lo_pair(c[8 * h + 2 * m], f[2 * m], c[8 * h + 2 * m + 1], f[2 * m + 1], H[m]);
  }
  hi = __builtin_bit_cast(f16x8, (u32x4){H[0], H[1], H[2], H[3]});
  lo = __builtin_bit_cast(f16x8, (u32x4){L[0], L[1], L[2], L[3]});
}
template <int N>
GDN_DEVICE void split_vec(const float* x, f16_t* hi, f16_t* lo) {
  static_assert(N % 2 == 0, "pairs");
#pragma unroll
  for (int m = 0; m < N; m += 2) split_pair(x[m], x[m + 1], hi[m], hi[m + 1], lo[m], lo[m + 1]);
}

// ---- T = (I + A)^-1 pieces ---------------------------------------------------------
//
// With A = strict_lower(beta_i k_i.k_j e^(gamma_i - gamma_j)), T = (I + A)^-1 is
// unit lower triangular and block lower triangular over the two 32-token
// halves, and its off-diagonal block satisfies
//   T_10 = -T_11 A_10 T_00,
// so each diagonal block is solved on its own (one wave each) and the
// off-diagonal block needs only the fp16 hi/lo of T_00, T_11 and A_10.  (beta
// scales the rows of R instead of the columns of T: with T' = T diag(beta)
// a small beta pushed T' into fp16's subnormal range, where its split lost
// precision.)

// fp32 working copy of a 32x32 diagonal block, kept in the two fp16 arrays
// of an off-diagonal block of the same T buffer: row i's columns 0..15 in
// the hi array, 16..31 in the lo array (64 bytes each, 8-byte aligned).
struct Scratch {
  // byte address of the block's row 0 in the hi array; the lo array follows
  // the hi array at a fixed distance, so a lane-dependent half is an integer
  // offset (a select between two pointers went through private memory and
  // turned the LDS accesses into flat ones)
  char* hi;
  static constexpr int kLoOff = C * LDH * (int)sizeof(f16_t);
  GDN_DEVICE float* row(int i, int half) const { return reinterpret_cast<float*>(hi + half * kLoOff + i * (2 * LDH)); }
  GDN_DEVICE float& at(int i, int j) const { return row(i, j >> 4)[j & 15]; }
};
static_assert(offsetof(TBuf, lo) == Scratch::kLoOff, "TBuf: lo follows hi");
// diagonal block blk (0 or 1) of tb is worked on in its off-diagonal block (0,1) or (1,0)
GDN_DEVICE Scratch scratch_of(TBuf& tb, int blk) {
  const int off = blk == 0 ? 32 : 32 * LDH;  // halves
  return {reinterpret_cast<char*>(tb.hi + off)};
}
GDN_DEVICE f32x4 load4(const float* p) {
  const f32x2 a = *reinterpret_cast<const f32x2*>(p), b = *reinterpret_cast<const f32x2*>(p + 2);
  return (f32x4){a[0], a[1], b[0], b[1]};
}

// 16x16 diagonal blocks of a 32x32 strictly lower block A (fp32) by
// right-looking forward substitution, in place: lane (b, c) = ((lane / 16) % 2,
// lane % 16) computes column c of block b; lanes 32..63 repeat lanes 0..31 and
// do not store.
GDN_DEVICE void invert_diag16(const Scratch& A, int lane) {
  const int b = (lane >> 4) & 1, c = lane & 15;
  float y[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) y[i] = i == c ? 1.f : 0.f;
#pragma unroll
  for (int kk = 0; kk < 15; ++kk) {
    const float xk = y[kk];
#pragma unroll
    for (int i = kk + 1; i < 16; ++i) y[i] = fmaf(-A.row(16 * b + i, b)[kk], xk, y[i]);
  }
  if (lane < 32) {
#pragma unroll
    for (int i = 0; i < 16; ++i) A.row(16 * b + i, b)[c] = y[i];
  }
}

GDN_DEVICE void split4(f32x4 x, f16x4& hi, f16x4& lo) {
  float xs[4] = {x[0], x[1], x[2], x[3]};
  f16_t h[4], l[4];
  split_vec<4>(xs, h, l);
  hi = (f16x4){h[0], h[1], h[2], h[3]};
  lo = (f16x4){l[0], l[1], l[2], l[3]};
}

// 16 -> 32 merge inside a 32x32 block whose diagonal 16-blocks hold their
// inverses: T_10 = -T_11 A_10 T_00, with 16x16x16 MFMAs on hi/lo splits.
GDN_DEVICE void merge16(const Scratch& A, int lane) {
  const int n = lane & 15, g4 = 4 * (lane >> 4);
  f16x4 ah, al, bh, bl;
  // M = A_10 T_00: A operand = rows of A_10, B operand = columns of T_00
  split4(load4(A.row(16 + n, 0) + g4), ah, al);
  {
    f32x4 y;
#pragma unroll
    for (int m = 0; m < 4; ++m) y[m] = A.row(g4 + m, 0)[n];
    split4(y, bh, bl);
  }
  f32x4 M = {0.f, 0.f, 0.f, 0.f};
  M = mfma16(ah, bh, M);
  M = mfma16(ah, bl, M);
  M = mfma16(al, bh, M);
  // T_10 = -T_11 M: A operand = rows of T_11, B operand = M (C layout rows == k)
  split4(load4(A.row(16 + n, 1) + g4), ah, al);
  split4(M, bh, bl);
  f32x4 R = {0.f, 0.f, 0.f, 0.f};
  R = mfma16(ah, bh, R);
  R = mfma16(ah, bl, R);
  R = mfma16(al, bh, R);
#pragma unroll
  for (int m = 0; m < 4; ++m) A.row(16 + g4 + m, 0)[n] = -R[m];
}

// Sequence of rank `rank` in longest-first order (ties by index); called by
// every thread of the block (the lengths are staged in T buffer 2, which is
// first written for chunk 2).
GDN_DEVICE int64_t seq_of_rank(Smem& sm, const PrefillArgs& a, int64_t rank, int tid) {
  if (a.nseq > kMaxRankedSeqs) return rank;
  static_assert(kMaxRankedSeqs * sizeof(int32_t) <= sizeof(TBuf), "lengths fit a T buffer");
  int32_t* lens = reinterpret_cast<int32_t*>(sm.tb[2].hi);
  for (int64_t i = tid; i < a.nseq; i += kThreads) {
    int64_t s, e;
    seq_range(a.cu, a.cu64, i, a.T, s, e);
    lens[i] = (int32_t)(e - s);
  }
  if (tid == 0) sm.seq = (int32_t)rank;
  __syncthreads();
  if (tid < a.nseq) {
    const int32_t li = lens[tid];
    int64_t rk = 0;
    for (int j = 0; j < a.nseq; ++j) {
      const int32_t lj = lens[j];
      rk += (lj > li) || (lj == li && j < tid);
    }
    if (rk == rank) sm.seq = tid;
  }
  __syncthreads();
  return sm.seq;
}

// ---- producer role (waves 4..7) --------------------------------------------------

// Producer barriers: LDS arrival counters that grow by the number of
// arriving waves per chunk.  A wave may arrive without waiting (its data is
// published by the release fence); waits are bounded so a logic error cannot
// hang the GPU.  A wait that gives up raises the workgroup's `failed` flag:
// the item then writes NaN to its output rows and leaves its state slot
// untouched, so a pipeline error fails loudly instead of giving a plausible
// answer.  (spin_limit is a kernel argument so that a test can force the
// give-up path from the host with every wave still exiting normally.)
GDN_DEVICE void producer_arrive(int32_t* count, int lane) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  if (lane == 0) __hip_atomic_fetch_add(count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
GDN_DEVICE void producer_wait(int32_t* count, int32_t target, int32_t spin_limit, int32_t* failed) {
  bool seen = false;
  for (int spin = 0; spin < spin_limit; ++spin) {
    if (__hip_atomic_load(count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) {
      seen = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  if (!seen) __hip_atomic_store(failed, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Where a (sequence, v-head) reads its chunks from.
struct ChunkSource {
  const PrefillArgs* a;
  const bf16_t* kg;  // k-head base
  const bf16_t* qg;  // k-head base
  const bf16_t* vg;  // v-head base
  int h;             // v-head
  int64_t e;         // end token of the sequence
};

GDN_DEVICE int chunk_rows(const ChunkSource& src, int64_t c0) {
  const int64_t rem = src.e - c0;
  return (int)(rem < C ? rem : C);
}

// Rows past the chunk's last token are loaded from the last token instead
// (no divergent loads, so nothing waits on them early): they are inert
// because their g, beta and e^(gamma_L - gamma) are set to zero, which zeroes
// their rows of R and their rows and columns of A (T keeps a unit row and
// column for them) and their share of the state update, and their output rows
// are not stored.
//
// 16 bytes of row `row` of a chunk (uniform base pointer of the chunk's first
// token + a 32-bit lane offset; the host guarantees 64 token strides fit).
GDN_DEVICE bf16x8 load_row_piece(const bf16_t* chunk_base, uint32_t stride, int row, int col, int Lc) {
  const uint32_t rc = (uint32_t)(row < Lc ? row : Lc - 1);
  const uint32_t byte_off = (rc * stride + (uint32_t)col) * (uint32_t)sizeof(bf16_t);
  return *reinterpret_cast<const bf16x8*>(reinterpret_cast<const char*>(chunk_base) + byte_off);
}

// A whole 64 x 128 chunk tile in one wave's registers: vector u of lane l is
// row l / 16 + 4u, columns 8 (l % 16) .. +7.
struct TileLoad {
  bf16x8 r[16];
};
// With a head dim below 128 (dim), a lane whose columns lie past it reads
// column 0 instead (in bounds); staging zeroes them.
GDN_DEVICE void load_tile(TileLoad& tl, const bf16_t* head_base, int64_t stride, int64_t c0, int Lc, int lane,
                          int dim = KD) {
  const bf16_t* b = head_base + c0 * stride;
  const int col = 8 * (lane & 15) < dim ? 8 * (lane & 15) : 0;
#pragma unroll
  for (int u = 0; u < 16; ++u) tl.r[u] = load_row_piece(b, (uint32_t)stride, (lane >> 4) + 4 * u, col, Lc);
}

// g and beta (raw bits) of token `lane` of a chunk.
struct DecayLoad {
  float g;
  ScalarRaw b;
};
GDN_DEVICE void load_decay(DecayLoad& dl, const ChunkSource& src, int64_t c0, int Lc, int lane) {
  const PrefillArgs& a = *src.a;
  const int64_t t = c0 + (lane < Lc ? lane : Lc - 1);
  dl.g = a.g[t * a.g_s0 + src.h * a.g_s1];
  dl.b = load_scalar_raw(a.beta, t * a.b_s0 + src.h * a.b_s1, a.b_dtype);
}

// K fragments of a diagonal block's 32 rows (lane (n, g) holds row 32 blk + n,
// columns 16 ks + 8 g .. +7) and the chunk's decays.
struct DiagLoad {
  bf16x8 kf[8];
  DecayLoad d;
};
GDN_DEVICE void load_diag(DiagLoad& dl, const ChunkSource& src, int64_t c0, int blk, int lane, int dim = KD) {
  const PrefillArgs& a = *src.a;
  const int Lc = chunk_rows(src, c0);
  const bf16_t* kb = src.kg + c0 * a.k_s0;
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const int col = 16 * ks + 8 * (lane >> 5);
    dl.kf[ks] = load_row_piece(kb, (uint32_t)a.k_s0, 32 * blk + (lane & 31), col < dim ? col : 0, Lc);
  }
  load_decay(dl.d, src, c0, Lc, lane);
}

// bf16 -> fp16 of 8 values (exact for |x| in the fp16 normal range): the
// bf16 bits widened to fp32 by a shift or mask, then one packed conversion
// per pair.
GDN_DEVICE f16x8 bf16x8_to_f16x8(bf16x8 x) {
  const u32x4 w = __builtin_bit_cast(u32x4, x);
  u32x4 o;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const f32x2 f = {__builtin_bit_cast(float, w[m] << 16), __builtin_bit_cast(float, w[m] & 0xffff0000u)};
    o[m] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2));
  }
  return __builtin_bit_cast(f16x8, o);
}

// The kernel reads q/k/v and writes o as 16-bit floats of one type: bf16
// (F16 = false) or fp16 (F16 = true).  Loads and the V tile move raw bits;
// these convert at the points of use.
template <bool F16>
GDN_DEVICE f16x8 to_f16x8(bf16x8 raw) {
  if constexpr (F16) return __builtin_bit_cast(f16x8, raw);
  else return bf16x8_to_f16x8(raw);
}
template <bool F16>
GDN_DEVICE f32x4 to_f32x4(s16x4 raw) {
  f32x4 r;
  if constexpr (F16) {
    const f16x4 h = __builtin_bit_cast(f16x4, raw);
#pragma unroll
    for (int m = 0; m < 4; ++m) r[m] = (float)h[m];
  } else {
    const bf16x4 h = __builtin_bit_cast(bf16x4, raw);
#pragma unroll
    for (int m = 0; m < 4; ++m) r[m] = (float)h[m];
  }
  return r;
}
template <bool F16>
GDN_DEVICE s16x4 from_f32x4(f32x4 x) {
  if constexpr (F16) {
    const f16x4 h = {(f16_t)x[0], (f16_t)x[1], (f16_t)x[2], (f16_t)x[3]};
    return __builtin_bit_cast(s16x4, h);
  } else {
    const bf16x4 h = {(bf16_t)x[0], (bf16_t)x[1], (bf16_t)x[2], (bf16_t)x[3]};
    return __builtin_bit_cast(s16x4, h);
  }
}

// gamma = in-chunk cumsum of g (one token per lane) and the per-token decay
// vectors; g and beta of tokens past the chunk end are taken as zero.
// Whether every lane's |gamma| < 80, so that e^gamma and e^-gamma are both
// normal floats and e^(gamma_i - gamma_j) = e^gamma_i e^-gamma_j loses nothing
// (one rounding per factor instead of an exponential per element).  Wave-uniform.
GDN_DEVICE bool factorable(float gm) {
  return __builtin_amdgcn_ballot_w64(!(fabsf(gm) < 80.f)) == 0;
}

GDN_DEVICE float chunk_gamma(const DecayLoad& dl, int L, int lane, float& gl) {
  const float gm = wave_inclusive_scan(lane < L ? dl.g : 0.f);
  gl = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gm), 63));  // gamma at token L-1
  return gm;
}

// Gram tile (mt, nt) of rows of M1 against rows of M2 (K = 128): C layout,
// lane holds column 32nt + n, rows 32mt + 8i + 4g + r.
GDN_DEVICE f32x16 gram_tile(const f16_t* M1, const f16_t* M2, int mt, int nt, int lane) {
  f32x16 G = zero16();
#pragma unroll
  for (int ks = 0; ks < KD / 16; ++ks)
    G = mfma32(frag_rows_kq(M1, 32 * mt, 16 * ks, lane), frag_rows_kq(M2, 32 * nt, 16 * ks, lane), G);
  return G;
}

// kk^T of a diagonal block's rows from the register fragments, in k's own
// 16-bit type (which holds k exactly)
template <bool F16>
GDN_DEVICE f32x16 gram_regs(const bf16x8 (&kf)[8]) {
  f32x16 G = zero16();
#pragma unroll
  for (int ks = 0; ks < KD / 16; ++ks) {
    if constexpr (F16) {
      const f16x8 h = __builtin_bit_cast(f16x8, kf[ks]);
      G = mfma32(h, h, G);
    } else {
      G = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], kf[ks], G, 0, 0, 0);
    }
  }
  return G;
}

// Diagonal block `blk` of T: A_bb = strict_lower(beta_i k_i.k_j e^(g_i - g_j))
// from its kk^T tile, solved in fp32 in the off-diagonal block of the same
// T buffer (16x16 substitution + one MFMA merge), then T_bb written as fp16
// hi/lo.  One wave, no workgroup synchronisation: the wave's
// LDS accesses complete in program order.  gam and beta: the chunk's vectors.
GDN_DEVICE void solve_diag_block(TBuf& tb, const float* gam, const float* beta, const float* eg, const float* ieg,
                                 bool fact, const f32x16& G, int blk, int lane) {
  const int n = lane & 31, gq = lane >> 5, o = 32 * blk;
  const Scratch A = scratch_of(tb, blk);
  if (fact) {
    const float ej = ieg[o + n];
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const f32x4 ei = rows4(eg, o, i4, lane);
      const f32x4 bi = rows4(beta, o, i4, lane);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int i = 8 * i4 + 4 * gq + rr;
        A.at(i, n) = i > n ? bi[rr] * G[4 * i4 + rr] * (ei[rr] * ej) : 0.f;
      }
    }
  } else {
    const float gj = gam[o + n];
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const f32x4 gi = rows4(gam, o, i4, lane);
      const f32x4 bi = rows4(beta, o, i4, lane);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int i = 8 * i4 + 4 * gq + rr;
        A.at(i, n) = i > n ? bi[rr] * G[4 * i4 + rr] * __expf(gi[rr] - gj) : 0.f;
      }
    }
  }
  invert_diag16(A, lane);
  merge16(A, lane);
  // T_bb (unit diagonal) as fp16 hi/lo: lane -> row lane / 2, 16 columns
  const int i = lane >> 1, half = lane & 1, j0 = 16 * half;
  float tv[16];
#pragma unroll
  for (int m = 0; m < 16; m += 4) {
    const f32x4 x = load4(A.row(i, half) + m);
#pragma unroll
    for (int z = 0; z < 4; ++z) tv[m + z] = x[z];
  }
  f16_t th[16], tl[16];
  split_vec<16>(tv, th, tl);
#pragma unroll
  for (int m = 0; m < 16; m += 4) {
    const int off = (o + i) * LDH + o + j0 + m;
    *reinterpret_cast<f16x4*>(tb.hi + off) = (f16x4){th[m], th[m + 1], th[m + 2], th[m + 3]};
    *reinterpret_cast<f16x4*>(tb.lo + off) = (f16x4){tl[m], tl[m + 1], tl[m + 2], tl[m + 3]};
  }
}

// A_10 = beta_i k_i.k_j e^(g_i - g_j) for tokens i in 32..63, j in 0..31
// (always i > j), as fp16 hi/lo in block (0,1) of the T arrays: A_10[i][j] at
// row i, column 32 + j.  |A_10| <= beta_i |k_i| |k_j| (<= 1 for unit keys and
// beta <= 1), split unscaled.
GDN_DEVICE void b10_block(const ChunkTiles& ct, TBuf& tb, int lane) {
  const int n = lane & 31, gq = lane >> 5;
  const f32x16 G = gram_tile(ct.k, ct.k, 1, 0, lane);
  float d[16];  // e^(gamma_i - gamma_j) for this lane's 16 entries
  if (__builtin_amdgcn_readfirstlane(ct.fact)) {
    const float ej = ct.ieg[n];
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const f32x4 ei = rows4(ct.eg, 32, i4, lane);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) d[4 * i4 + rr] = ei[rr] * ej;
    }
  } else {
    const float gj = ct.gam[n];
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const f32x4 gi = rows4(ct.gam, 32, i4, lane);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) d[4 * i4 + rr] = __expf(gi[rr] - gj);
    }
  }
#pragma unroll
  for (int i4 = 0; i4 < 4; ++i4) {
    const f32x4 bi = rows4(ct.beta, 32, i4, lane);
#pragma unroll
    for (int rr = 0; rr < 4; rr += 2) {
      const int i = 8 * i4 + 4 * gq + rr;
      f16_t h0, h1, l0, l1;
      split_pair(G[4 * i4 + rr] * (d[4 * i4 + rr] * bi[rr]), G[4 * i4 + rr + 1] * (d[4 * i4 + rr + 1] * bi[rr + 1]),
                 h0, h1, l0, l1);
      tb.hi[i * LDH + 32 + n] = h0;
      tb.hi[(i + 1) * LDH + 32 + n] = h1;
      tb.lo[i * LDH + 32 + n] = l0;
      tb.lo[(i + 1) * LDH + 32 + n] = l1;
    }
  }
}

// T_10 = -T_11 A_10 T_00 from the fp16 hi/lo blocks (lo x lo dropped).  One wave.
GDN_DEVICE void merge_offdiag(TBuf& tb, int lane) {
  const int n = lane & 31, gq = lane >> 5;
  const f16_t* th = tb.hi;
  const f16_t* tl = tb.lo;
  // M = A_10 T_00: A operand = rows of A_10, B operand = columns of T_00
  f32x16 M = zero16();
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const f16x8 bh = frag_rows(th, LDH, 0, 32 + 16 * ks, lane), bl = frag_rows(tl, LDH, 0, 32 + 16 * ks, lane);
    const f16x8 ch = frag_cols(th, LDH, 0, 16 * ks, lane), cl = frag_cols(tl, LDH, 0, 16 * ks, lane);
    M = mfma32(bh, ch, M);
    M = mfma32(bh, cl, M);
    M = mfma32(bl, ch, M);
  }
  // -T_11 M: A operand = rows of T_11, B operand = M (C layout rows == k)
  f32x16 R = zero16();
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const f16x8 ah = frag_rows(th, LDH, 32, 32 + 16 * ks, lane), al = frag_rows(tl, LDH, 32, 32 + 16 * ks, lane);
    f16x8 mh, ml;
    split8(M, ks, 1.f, mh, ml);
    R = mfma32(ah, mh, R);
    R = mfma32(ah, ml, R);
    R = mfma32(al, mh, R);
  }
#pragma unroll
  for (int j = 0; j < 16; j += 2) {
    const int i = 32 + 8 * (j >> 2) + 4 * gq + (j & 3);
    f16_t h0, h1, l0, l1;
    split_pair(-R[j], -R[j + 1], h0, h1, l0, l1);
    tb.hi[i * LDH + n] = h0;
    tb.hi[(i + 1) * LDH + n] = h1;
    tb.lo[i * LDH + n] = l0;
    tb.lo[(i + 1) * LDH + n] = l1;
  }
}

// (Q K^T) tile (mt, nt) -> P = lower(q_i.k_j e^(g_i - g_j)) as fp16, C layout
// (element 4 i4 + rr of the tile at row 32mt + 8 i4 + 4g + rr).
GDN_DEVICE f16x8 qk_half(const f32x16& G, const ChunkTiles& ct, bool fact, int mt, int nt, int h, int lane) {
  const int n = lane & 31, gq = lane >> 5;
  const int j = 32 * nt + n;
  f16x8 out;
  if (fact) {
    const float ej = ct.ieg[j];
#pragma unroll
    for (int i4 = 2 * h; i4 < 2 * h + 2; ++i4) {
      const f32x4 ei = rows4(ct.eg, 32 * mt, i4, lane);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int i = 32 * mt + 8 * i4 + 4 * gq + rr;
        out[4 * (i4 - 2 * h) + rr] = (f16_t)(i >= j ? G[4 * i4 + rr] * (ei[rr] * ej) : 0.f);
      }
    }
  } else {
    const float gj = ct.gam[j];
#pragma unroll
    for (int i4 = 2 * h; i4 < 2 * h + 2; ++i4) {
      const f32x4 gi = rows4(ct.gam, 32 * mt, i4, lane);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int i = 32 * mt + 8 * i4 + 4 * gq + rr;
        out[4 * (i4 - 2 * h) + rr] = (f16_t)(i >= j ? G[4 * i4 + rr] * __expf(gi[rr] - gj) : 0.f);
      }
    }
  }
  return out;
}
GDN_DEVICE void p_tile(ChunkTiles& ct, int mt, int nt, int lane) {
  const f32x16 G = gram_tile(ct.q, ct.k, mt, nt, lane);
  const bool fact = __builtin_amdgcn_readfirstlane(ct.fact) != 0;
  const f16x8 h0 = qk_half(G, ct, fact, mt, nt, 0, lane), h1 = qk_half(G, ct, fact, mt, nt, 1, lane);
  const int n = lane & 31, gq = lane >> 5;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int i = 32 * mt + 8 * (e >> 2) + 4 * gq + (e & 3);
    ct.p[i * LDH + 32 * nt + n] = e < 8 ? h0[e] : h1[e - 8];
  }
}

// Stage a tile held in registers into LDS (fp16 for K/Q, the raw 16-bit
// elements for V).
template <bool F16>
GDN_DEVICE void stage_f16(f16_t* dst, const TileLoad& tl, int lane, bool keep = true) {
  // lane's 8 logical columns 8a..8a+7 (a = lane % 16) are quads 2a', 2a'+1 of
  // 16-column group a / 2 (a' = a % 2), stored at quads kq_quad(2a'), kq_quad(2a'+1)
  const int a = lane & 15, grp = 16 * (a >> 1), q0 = 2 * (a & 1);
  const int off0 = grp + 4 * kq_quad(q0), off1 = grp + 4 * kq_quad(q0 + 1);
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const f16x8 v = keep ? to_f16x8<F16>(tl.r[u]) : f16x8{};  // (keep: the lane's columns lie inside the head dim)
    f16_t* row = dst + ((lane >> 4) + 4 * u) * LDK;
    *reinterpret_cast<f16x4*>(row + off0) = (f16x4){v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f16x4*>(row + off1) = (f16x4){v[4], v[5], v[6], v[7]};
  }
}
GDN_DEVICE void stage_v(bf16_t* dst, const TileLoad& tl, int lane, bool keep = true) {
#pragma unroll
  for (int u = 0; u < 16; ++u)
    *reinterpret_cast<bf16x8*>(dst + ((lane >> 4) + 4 * u) * LDV + 8 * (lane & 15)) = keep ? tl.r[u] : bf16x8{};
}

// Decay vectors of a chunk for the state waves and the producers' epilogues.
GDN_DEVICE void stage_decay(ChunkTiles& ct, const DecayLoad& dl, int L, int b_dtype, int lane) {
  float gl;
  const float gm = chunk_gamma(dl, L, lane, gl);
  ct.gam[lane] = gm;
  ct.eg[lane] = __expf(gm);
  ct.ieg[lane] = __expf(-gm);
  const bool fact = factorable(gm);
  if (lane == 0) ct.fact = fact;
  ct.edec[lane] = lane < L ? __expf(gl - gm) : 0.f;
  ct.beta[lane] = lane < L ? scalar_raw_f32(dl.b, b_dtype) : 0.f;
  if (lane == 0) ct.gam_last = gl;
}

// ---- state role (waves 0..3) -----------------------------------------------------

// Slot (0..7, 4 rows each) of a 32-row half of output column m in the output
// staging: slot s is permuted by m / 4 with bits 1 and 2 of m / 4 swapped, so
// the 32 columns of one 8-byte write and the column groups of one transposed
// read each land in distinct banks.
GDN_DEVICE int out_slot(int s, int m) {
  const int q = (m >> 2) & 7;
  return s ^ (((q & 2) << 1) | ((q & 4) >> 1) | (q & 1));
}

// The state products of one chunk on this wave's 32 value columns; writes the
// chunk's output rows for those columns (16-bit outputs are staged through its
// own columns of the V tile, fp32 outputs (OUT32) are stored straight from the
// accumulators; then it signals v_free).  The state is held in units of
// 2^su (true state = S * 2^su; su is per value column, since no product
// mixes value columns): the update rescales S by one factor per chunk and
// picks the new units from the exponents of V' and of the decayed state, so
// S stays below 2^14 and is split without another pass over it.
template <bool F16, bool PAD, bool OUT32>
GDN_DEVICE void consume_chunk(const ChunkTiles& ct, const TBuf& tb, float kn2, bf16_t* vt, int32_t* v_free,
                              f32x16 (&S)[4], int& su, float& sb, const PrefillArgs& a, int64_t c0, int L, int h,
                              int wave, int lane) {
  // Lane-dependent addresses are cheap to recompute; keeping them out of
  // loop-invariant code motion keeps them out of registers across chunks.
  asm volatile("" : "+v"(lane));
  const int n = lane & 31, gq = lane >> 5;
  // X = K S, QS = Q S on the split of S itself (the choice of units below
  // keeps |S| < 2^14, so fp16 cannot overflow; true values: X 2^su)
  f32x16 X[2] = {zero16(), zero16()}, QS[2] = {zero16(), zero16()};
  float one = 1.f;  // opaque, so lo = fp16(fma(x, one, -hi)) stays one mixed-precision fma
  asm volatile("" : "+v"(one));
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    f16x8 shi, slo;
    split8u(S[ks >> 1], ks & 1, one, shi, slo);
    const f16x8 ak0 = frag_rows_kq(ct.k, 0, 16 * ks, lane);
    const f16x8 ak1 = frag_rows_kq(ct.k, 32, 16 * ks, lane);
    const f16x8 aq0 = frag_rows_kq(ct.q, 0, 16 * ks, lane);
    const f16x8 aq1 = frag_rows_kq(ct.q, 32, 16 * ks, lane);
    X[0] = mfma32(ak0, shi, X[0]);
    X[1] = mfma32(ak1, shi, X[1]);
    QS[0] = mfma32(aq0, shi, QS[0]);
    QS[1] = mfma32(aq1, shi, QS[1]);
    X[0] = mfma32(ak0, slo, X[0]);
    X[1] = mfma32(ak1, slo, X[1]);
  }
  const int ex = su;
  // exponent of a bound of this column's state maximum (max |S| <= sb < 2^sm), for the next units
  const int sm = sb > 0.f ? __builtin_amdgcn_frexp_expf(sb) : kNone;
  // R = diag(beta) (V - diag(e^gamma) X) in true units (V read transposed:
  // rows are tokens); beta multiplies R rather than T, so T keeps its unit
  // diagonal and its fp16 split keeps full precision for any beta
  const float xu = __builtin_amdgcn_ldexpf(1.f, ex);
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 egv = rows4(ct.eg, 32 * mt, i, lane);
      const f32x4 bv = rows4(ct.beta, 32 * mt, i, lane);
      const int j = lane & 15, qd = lane >> 4;
      const bf16_t* p = vt + (32 * mt + 8 * i + 4 * (qd >> 1) + (j >> 2)) * LDV + 32 * wave + 16 * (qd & 1) + 4 * (j & 3);
      const f32x4 vv = to_f32x4<F16>(tr_read(p));
      // (v - e^gamma 2^su X) first, in one fma, then times beta: one multiply
      // per element less than scaling both terms by beta, and the cancellation
      // happens before any rounding
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) X[mt][4 * i + rr] = bv[rr] * fmaf(-(egv[rr] * xu), X[mt][4 * i + rr], vv[rr]);
    }
  }
  f32x16* R = X;  // X now holds R
  // (er >= ex - 100 keeps 2^(ex - er) finite; a smaller R is negligible next to the state)
  const int er = max(col_scale_exp(R, 2), ex - 100);
  const float rs = __builtin_amdgcn_ldexpf(1.f, -er);
  // V' = T R, in units of 2^er (T lower triangular: rows 0..31 need only k-steps 0, 1)
  f32x16 VN[2] = {zero16(), zero16()};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    f16x8 rhi, rlo;
    split8(R[ks >> 1], ks & 1, rs, rhi, rlo);
    if (ks < 2) {
      const f16x8 ah0 = frag_rows(tb.hi, LDH, 0, 16 * ks, lane);
      const f16x8 al0 = frag_rows(tb.lo, LDH, 0, 16 * ks, lane);
      const f16x8 ah1 = frag_rows(tb.hi, LDH, 32, 16 * ks, lane);
      const f16x8 al1 = frag_rows(tb.lo, LDH, 32, 16 * ks, lane);
      VN[0] = mfma32(ah0, rhi, VN[0]);
      VN[1] = mfma32(ah1, rhi, VN[1]);
      VN[0] = mfma32(ah0, rlo, VN[0]);
      VN[1] = mfma32(ah1, rlo, VN[1]);
      VN[0] = mfma32(al0, rhi, VN[0]);
      VN[1] = mfma32(al1, rhi, VN[1]);
    } else {
      const f16x8 ah1 = frag_rows(tb.hi, LDH, 32, 16 * ks, lane);
      const f16x8 al1 = frag_rows(tb.lo, LDH, 32, 16 * ks, lane);
      VN[1] = mfma32(ah1, rhi, VN[1]);
      VN[1] = mfma32(ah1, rlo, VN[1]);
      VN[1] = mfma32(al1, rhi, VN[1]);
    }
  }
  // O = scale (diag(e^gamma) Q S + P V') = scale 2^er (diag(e^gamma 2^(ex - er)) QS + P VN)
  const float qsu = __builtin_amdgcn_ldexpf(1.f, ex - er);
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 egv = rows4(ct.eg, 32 * mt, i, lane);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) QS[mt][4 * i + rr] *= egv[rr] * qsu;
    }
  }
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    f16x8 vb;
#pragma unroll
    for (int m = 0; m < 8; ++m) vb[m] = (f16_t)VN[ks >> 1][8 * (ks & 1) + m];
#pragma unroll
    for (int mt = (ks >> 1); mt < 2; ++mt) QS[mt] = mfma32(frag_rows(ct.p, LDH, 32 * mt, 16 * ks, lane), vb, QS[mt]);
  }
  if constexpr (OUT32) {
    // fp32 output straight from the accumulators: lane (n, g) holds column
    // 32 wave + n of rows 32 mt + 8 i + 4 g + rr; one store instruction
    // covers 32 consecutive columns of two rows.  GDN_PREFILL_ACCUM_OUT adds
    // to what out holds.
    const float osc = __builtin_amdgcn_ldexpf(a.scale, er);
    const bool acc = (a.flags & GDN_PREFILL_ACCUM_OUT) != 0;
    float* ob = reinterpret_cast<float*>(a.out) + c0 * a.o_s0 + h * a.o_s1 + 32 * wave + n;
    if (!PAD || 32 * wave + n < a.vd) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const int row = 32 * mt + 8 * i + 4 * gq + rr;
            if (row < L) {
              float* p = ob + (uint32_t)row * (uint32_t)a.o_s0;
              const float o = QS[mt][4 * i + rr] * osc;
              *p = acc ? *p + o : o;
            }
          }
    }
  } else {
  // Stage this wave's output columns (bf16) in its own columns of the V tile,
  // column-major: output column m's rows 32 h .. 32 h + 31 sit in tile row
  // 2 m + h, in eight 4-row slots permuted by out_slot (conflict-free 8-byte
  // writes and transposed reads).  Each lane writes 4 consecutive rows of its
  // column at once, then reads back 16-byte row pieces with transposed reads.
    const float osc = __builtin_amdgcn_ldexpf(a.scale, er);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4 o4;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) o4[rr] = QS[mt][4 * i + rr] * osc;
        *reinterpret_cast<s16x4*>(vt + (2 * n + mt) * LDV + 32 * wave + 4 * out_slot(2 * i + gq, n)) = from_f32x4<F16>(o4);
      }
    // lane (qd, j) of the four 16-lane groups: output row 16 u + j, columns 8 qd .. 8 qd + 7
    const int j = lane & 15, qd = lane >> 4;
    bf16_t* ob = a.out + c0 * a.o_s0 + h * a.o_s1 + 32 * wave + 8 * qd;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      s16x4 half[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int m = 8 * qd + 4 * hh + (j >> 2);  // output column of this lane's address
        half[hh] = tr_read(vt + (2 * m + (u >> 1)) * LDV + 32 * wave + 4 * out_slot(4 * (u & 1) + (j & 3), m));
      }
      const int row = 16 * u + j;
      if (row < L && (!PAD || 32 * wave + 8 * qd < a.vd))
        *reinterpret_cast<u32x4*>(reinterpret_cast<char*>(ob) + (uint32_t)row * (uint32_t)a.o_s0 * 2u) =
            __builtin_bit_cast(u32x4, (s16x8){half[0][0], half[0][1], half[0][2], half[0][3],
                                               half[1][0], half[1][1], half[1][2], half[1][3]});
    }
  }
  // this wave is done with the V tile (its values, then its output staging)
  producer_arrive(v_free, lane);
  // S_true' = e^gamma_L S_true + K^T Vd, Vd = diag(e^(gamma_L - gamma)) V' = diag(edec) VN 2^er,
  // with the new state in units of 2^ed:  S' = S e^gamma_L 2^(su - ed) + K^T (Vd 2^-ed).
  // ed keeps the split of S' (next chunk, unscaled) inside the fp16 range:
  //  * the update: with max |VN| < 2^vm and edec <= 1 the split operand
  //    Vd 2^-ed is below 2^(vm + er - ed), and entry (i, j) of the update is
  //    below 2^(vm + er - ed) sum_t |k_t,i| <= 2^(vm + er - ed) kb with
  //    kb = 64 max_t |k_t| (the chunk's largest key norm, from the Gram
  //    diagonal), so it is below 2^12 when ed >= er + vm + kbe - 12
  //    (kb <= 2^kbe; kbe = 6 or 7 for L2-normalised keys);
  //  * the decayed state: with max |S| < 2^sm and e^gamma_L < 2^lm it is below
  //    2^(sm + lm + su - ed) <= 2^13 when ed >= sm + lm + su - 13;
  // so |S'| < 2^13 + 2^12 for keys of any norm.  A part that is zero (sm, vm,
  // lm or kbe = kNone) sets no bound; ed >= er - 100 keeps 2^(er - ed) finite.
  const float edl = __expf(ct.gam_last);
  const int vm = col_max_exp(VN, 2);
  const int lm = edl > 0.f ? __builtin_amdgcn_frexp_expf(edl) : kNone;
  const float kb = 64.f * __builtin_sqrtf(kn2);
  const int kbe = kb > 0.f ? __builtin_amdgcn_frexp_expf(kb) : kNone;
  const int ed = max(max(er + vm + kbe - 12, sm + lm + su - 13), er - 100);
  const float fdu = __builtin_amdgcn_ldexpf(1.f, er - ed);
  // U = K^T (Vd 2^-ed) from zero accumulators, then S' = S e^gamma_L 2^(su - ed) + U
  // (one fma per element; the MFMAs need not wait for the decay, and the state
  // is not carried through the accumulator tuples, which cost a register copy
  // of all 64 values per chunk)
  f32x16 U[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    float fd[8];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const f32x4 dv = rows4(ct.edec, 32 * (ks >> 1), 2 * (ks & 1) + i, lane);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) fd[4 * i + rr] = dv[rr] * fdu;
    }
    f16x8 dhi, dlo;
    split8f(VN[ks >> 1], ks & 1, fd, dhi, dlo);
    f16x8 akt[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) akt[mt] = frag_cols_kq(ct.k, 32 * mt, 16 * ks, lane);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) U[mt] = mfma32(akt[mt], dhi, ks == 0 ? zero16() : U[mt]);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) U[mt] = mfma32(akt[mt], dlo, U[mt]);
  }
  const int dsu = su - ed;
  float sdec = __builtin_amdgcn_ldexpf(edl, dsu);  // 0 when it underflows: the old state is negligible then
  // bound of the new column maximum: the decayed bound plus the update's (|U| < 2^(vm + er - ed) kb)
  const float ub = vm == kNone ? 0.f : __builtin_amdgcn_ldexpf(kb, vm + er - ed);
  float sbd = sb * sdec;
  if (__builtin_amdgcn_ballot_w64(!(sdec <= 3.0e38f)) != 0) {
    // the factor overflows on some column: scale element by element first
    // (the empty asm keeps this rare path out of the common one)
    asm volatile("");
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int j = 0; j < 16; ++j) S[mt][j] = __builtin_amdgcn_ldexpf(S[mt][j] * edl, dsu);
    sdec = 1.f;
    sbd = __builtin_amdgcn_ldexpf(sb * edl, dsu);
  }
  sb = sbd + ub;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int j = 0; j < 16; ++j) S[mt][j] = fmaf(S[mt][j], sdec, U[mt][j]);
  su = ed;
}

// ---- the workgroup's items and its chunk stream -------------------------------
//
// A workgroup processes one item (sequence, v-head) or, for batches of many
// short sequences, up to 64 consecutive items: item j's fields sit in lane j
// of every wave and are read with readlane.  All roles walk the same stream of
// (item, chunk) positions, so the producers stage and solve the next item's
// first chunks while the state waves still work on the current item.
struct Items {
  int64_t s, e;  // token range of the lane's item
  int32_t slot;  // its state slot, -1 for a padding sequence
  int32_t h;     // its v-head
  int32_t nc;    // its chunks (0: empty or padding, no state work)
  int m;         // items of the workgroup (uniform)
};
GDN_DEVICE int32_t rd32(int32_t x, int j) { return __builtin_amdgcn_readlane(x, j); }
GDN_DEVICE int64_t rd64(int64_t x, int j) {
  const uint64_t u = (uint64_t)x;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int32_t)(uint32_t)u, j);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int32_t)(uint32_t)(u >> 32), j);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
// Position in the stream: chunk c of item j (j == m: past the end).
struct Pos {
  int j, c;
};
GDN_DEVICE Pos skip_empty(const Items& it, Pos p) {
  while (p.j < it.m && rd32(it.nc, p.j) == 0) ++p.j;
  return p;
}
GDN_DEVICE Pos next_pos(const Items& it, Pos p) {
  if (++p.c >= rd32(it.nc, p.j)) {
    p.c = 0;
    ++p.j;
    p = skip_empty(it, p);
  }
  return p;
}
struct ChunkAt {
  int64_t c0, e;  // first token of the chunk, end of its sequence
  int L, h;       // tokens in the chunk, v-head
  int32_t slot;
};
GDN_DEVICE ChunkAt chunk_at(const Items& it, Pos p) {
  ChunkAt ch;
  ch.e = rd64(it.e, p.j);
  ch.c0 = rd64(it.s, p.j) + (int64_t)p.c * C;
  const int64_t r = ch.e - ch.c0;
  ch.L = (int)(r < C ? r : C);
  ch.h = rd32(it.h, p.j);
  ch.slot = rd32(it.slot, p.j);
  return ch;
}
GDN_DEVICE ChunkSource source_of(const PrefillArgs& a, const ChunkAt& ch) {
  const int kh = ch.h / a.r;
  return {&a, a.k + kh * a.k_s1, a.q + kh * a.q_s1, a.v + ch.h * a.v_s1, ch.h, ch.e};
}
// Item fields of (sequence, v-head) = (seq, h).
GDN_DEVICE void item_fields(const PrefillArgs& a, int64_t seq, int h, Items& it) {
  seq_range(a.cu, a.cu64, seq, a.T, it.s, it.e);
  const int64_t slot = load_index(a.idx, seq, a.idx64);
  const bool pad = slot < 0 || slot >= a.num_slots;
  it.slot = pad ? -1 : (int32_t)slot;
  it.h = h;
  it.nc = (pad || it.e <= it.s) ? 0 : (int32_t)((it.e - it.s + C - 1) / C);
}

// ---- several items per workgroup: runs of work ids dealt by cost ------------
//
// Work ids are sequence-major (w = sequence * Hv + v-head), so the v-heads of
// a k-head, and all heads of a sequence, are neighbours.  An item is priced
// at its token count plus kItemCost tokens (what an item boundary costs: the
// state store and the next state's load take about 0.6 of a 64-token chunk
// step), and workgroup b of nwg takes the items whose price interval starts
// in [b P / nwg, (b + 1) P / nwg), P the batch's total price.  Prices are a
// closed form of cu_seqlens, so every wave finds its run's ends by two
// searches over cu_seqlens, with no pass over the batch and no host sync; a
// long sequence among many short ones is thereby spread over workgroups
// instead of sharing one with all of its v-heads.
constexpr int64_t kItemCost = 40;

// Price of the items before sequence s, per v-head (cu clamped like seq_range).
GDN_DEVICE int64_t price_before(const PrefillArgs& a, int64_t s) {
  int64_t c0 = load_index(a.cu, 0, a.cu64), cs = load_index(a.cu, s, a.cu64);
  c0 = c0 < 0 ? 0 : (c0 > a.T ? a.T : c0);
  cs = cs < c0 ? c0 : (cs > a.T ? a.T : cs);
  return (cs - c0) + kItemCost * s;
}

// First work id whose price interval starts at or after `target` (all lanes
// of the wave take part; a 64-ary search over the sequences, one probe per
// lane per round, so two rounds cover 4096 sequences).
GDN_DEVICE int64_t first_item_at(const PrefillArgs& a, int64_t target, int lane) {
  const int64_t Hv = a.Hv;
  // largest s in [0, nseq] with Hv * price_before(s) <= target (true at s = 0)
  int64_t lo = 0, span = a.nseq + 1;
  while (span > 1) {
    const int64_t step = (span + 63) / 64;
    const int64_t s = lo + lane * step;
    const int64_t sl = s < a.nseq ? s : a.nseq;  // (every lane loads inside cu_seqlens)
    const bool ok = s < lo + span && Hv * price_before(a, sl) <= target;
    const int cnt = __builtin_popcountll(__builtin_amdgcn_ballot_w64(ok));  // >= 1: lane 0 probes lo
    const int64_t nlo = lo + (int64_t)(cnt - 1) * step;
    span = (lo + span - nlo) < step ? (lo + span - nlo) : step;
    lo = nlo;
  }
  if (lo >= a.nseq) return a.nseq * Hv;
  const int64_t p0 = Hv * price_before(a, lo);
  const int64_t c = price_before(a, lo + 1) - price_before(a, lo);  // >= kItemCost
  const int64_t h = (target - p0 + c - 1) / c;  // first v-head of sequence lo starting at or after target
  return h >= Hv ? (lo + 1) * Hv : lo * Hv + h;
}

// This workgroup's run [w0, w1) of work ids; workgroup b's w1 is workgroup
// b + 1's w0 (the same expression), so the runs tile [0, nseq Hv).
GDN_DEVICE void multi_run(const PrefillArgs& a, int64_t bid, int64_t nwg, int lane, int64_t& w0, int64_t& w1) {
  const int64_t total = a.Hv * price_before(a, a.nseq);
  const int64_t q = total / nwg, r = total % nwg;
  auto target = [&](int64_t b) { return q * b + (r * b) / nwg; };  // floor(total b / nwg) without overflow
  w0 = bid == 0 ? 0 : first_item_at(a, target(bid), lane);
  w1 = bid + 1 >= nwg ? a.nseq * a.Hv : first_item_at(a, target(bid + 1), lane);
}

// All roles walk the chunk stream of the items in `it` (every role executes
// exactly 1 + nq workgroup barriers, nq = chunks in the stream).
// PAD: head dims below 128, zero-padded to 128 in the tiles and the state
// registers (zero key columns and zero value columns leave the rest exact).
// OUT32: fp32 output (q, k, v fp16).
template <bool F16, bool MULTI, bool PAD, bool OUT32>
GDN_DEVICE void run_items(Smem& sm, const PrefillArgs& a, const Items& it, int tid) {
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // (uniform: role branches and per-wave offsets in scalar registers)
  // padding sequences: zero output rows, no state (GDN_PREFILL_ACCUM_OUT: nothing to add)
  constexpr int kVec = OUT32 ? 4 : 8;  // output elements per 16-byte vector
  constexpr int kLanesPerRow = VD / kVec;
  for (int j = 0; j < it.m; ++j) {
    if (rd32(it.slot, j) >= 0 || (a.flags & GDN_PREFILL_ACCUM_OUT)) continue;
    const int64_t s = rd64(it.s, j), e = rd64(it.e, j);
    const int h = rd32(it.h, j);
    const int col = kVec * (tid % kLanesPerRow);
    if (PAD && col >= a.vd) continue;  // (no barrier or cross-lane step follows in this loop)
    for (int64_t t = s + tid / kLanesPerRow; t < e; t += kThreads / kLanesPerRow) {
      char* p = reinterpret_cast<char*>(a.out) + (t * a.o_s0 + h * a.o_s1 + col) * (OUT32 ? 4 : 2);
      *reinterpret_cast<u32x4*>(p) = u32x4{0u, 0u, 0u, 0u};
    }
  }
  int nq = 0;  // chunks in the stream
  for (int j = 0; j < it.m; ++j) nq += rd32(it.nc, j);
  if (nq == 0) return;
  const Pos first = skip_empty(it, Pos{0, 0});

  // Every role executes exactly 1 + nq workgroup barriers.
  if (wave < 4) {
    // ---- state waves: S (K x V fp32) in C layout, m-tile mt = keys 32mt.., this wave's 32 columns
    // (lane (n, g) holds column 32 wave + n, keys 32mt + 8 (j / 4) + 4g + j % 4)
    f32x16 S[4];
    int su = 0;
    float sb = 0.f;  // upper bound of the column's max |S|, carried across chunks
    auto state_of = [&](const ChunkAt& ch) __attribute__((always_inline)) {
      return a.state + (int64_t)ch.slot * a.st_slot + ch.h * a.st_head;
    };
    // (the state's lane offsets are recomputed at each load and store rather
    // than held in registers across the chunk loop)
    auto load_state = [&](const ChunkAt& ch) __attribute__((always_inline)) {
      if (a.flags & GDN_PREFILL_ZERO_INIT) {  // start from zero; the slot is not read
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) S[mt] = zero16();
        su = 0;
        sb = 0.f;
        return;
      }
      int ln = lane;
      asm volatile("" : "+v"(ln));
      if constexpr (PAD) {
        // rows of a.vd values; keys past a.kd and values past a.vd are zero
        const float* Sb = state_of(ch);
        const int c = 32 * wave + (ln & 31);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int r = 32 * mt + 8 * (j >> 2) + (j & 3) + 4 * (ln >> 5);
            const bool in = r < a.kd && c < a.vd;
            const float x = Sb[in ? r * a.vd + c : 0];
            S[mt][j] = in ? x : 0.f;
          }
      } else {
        const float* Sg = state_of(ch) + (4 * (ln >> 5)) * VD + 32 * wave + (ln & 31);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int j = 0; j < 16; ++j) S[mt][j] = Sg[(32 * mt + 8 * (j >> 2) + (j & 3)) * VD];
      }
      // state units: true state = S * 2^su, with |S| < 2^10 to start with
      const int sme = col_max_exp(S, 4);
      su = sme == kNone ? 0 : sme - 10;
      sb = sme == kNone ? 0.f : 1024.f;
      const float f = __builtin_amdgcn_ldexpf(1.f, -su);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int j = 0; j < 16; ++j) S[mt][j] *= f;
    };
    Pos p = first;
    load_state(chunk_at(it, p));
    __syncthreads();  // chunk 0 is prepared
    for (int q = 0; q < nq; ++q) {
      const ChunkAt ch = chunk_at(it, p);
      consume_chunk<F16, PAD, OUT32>(sm.tiles[q & 1], sm.tb[q % 3], fmaxf(sm.kn2[q % 3][0], sm.kn2[q % 3][1]), sm.v, &sm.v_free,
                         S, su, sb, a, ch.c0, ch.L, ch.h, wave, lane);
      // the carried bound only grows looser: every 16 chunks it is replaced by the exact maximum
      if ((p.c & 15) == 15) sb = col_max(S, 4);
      const Pos pn = next_pos(it, p);
      if (pn.j != p.j) {
        // the item's last chunk: its state goes back to its slot, or, if a
        // producer wait gave up, NaN in every output row of the item (this
        // wave's 32 columns) and the slot untouched (the flag stays raised, so
        // every later item of the workgroup fails the same way)
        const int64_t s0 = rd64(it.s, p.j);
        if (__hip_atomic_load(&sm.failed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0) {
          // (the NaN is made opaque here so that it is not materialised, and
          // kept in registers, ahead of the chunk loop)
          float nan = __builtin_nanf("");
          asm volatile("" : "+v"(nan));
          if constexpr (OUT32) {
            if (!PAD || 32 * wave + 4 * (lane & 7) < a.vd)
              for (int64_t t = s0 + (lane >> 3); t < ch.e; t += 8)
                *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.out) + t * a.o_s0 + ch.h * a.o_s1 + 32 * wave +
                                          4 * (lane & 7)) = f32x4{nan, nan, nan, nan};
          } else {
            const s16x4 nan4 = from_f32x4<F16>((f32x4){nan, nan, nan, nan});
            const bf16x8 z = __builtin_bit_cast(bf16x8, (s16x8){nan4[0], nan4[1], nan4[2], nan4[3],
                                                                nan4[0], nan4[1], nan4[2], nan4[3]});
            if (!PAD || 32 * wave + 8 * (lane & 3) < a.vd)
              for (int64_t t = s0 + (lane >> 2); t < ch.e; t += 16)
                *reinterpret_cast<bf16x8*>(a.out + t * a.o_s0 + ch.h * a.o_s1 + 32 * wave + 8 * (lane & 3)) = z;
          }
        } else {
          // the final state goes back to the slot (GDN_PREFILL_ACCUM_STATE: is added to it)
          const bool acc = (a.flags & GDN_PREFILL_ACCUM_STATE) != 0;
          int ln = lane;
          asm volatile("" : "+v"(ln));
          if constexpr (PAD) {
            float* Sb = state_of(ch);
            const int c = 32 * wave + (ln & 31);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
              for (int j = 0; j < 16; ++j) {
                const int r = 32 * mt + 8 * (j >> 2) + (j & 3) + 4 * (ln >> 5);
                if (r < a.kd && c < a.vd) {
                  const float x = __builtin_amdgcn_ldexpf(S[mt][j], su);
                  Sb[r * a.vd + c] = acc ? Sb[r * a.vd + c] + x : x;
                }
              }
          } else if (acc) {
            asm volatile("");
            float* Sg = state_of(ch) + (4 * (ln >> 5)) * VD + 32 * wave + (ln & 31);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
              for (int j = 0; j < 16; ++j)
                Sg[(32 * mt + 8 * (j >> 2) + (j & 3)) * VD] += __builtin_amdgcn_ldexpf(S[mt][j], su);
          } else {
            float* Sg = state_of(ch) + (4 * (ln >> 5)) * VD + 32 * wave + (ln & 31);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
              for (int j = 0; j < 16; ++j)
                Sg[(32 * mt + 8 * (j >> 2) + (j & 3)) * VD] = __builtin_amdgcn_ldexpf(S[mt][j], su);
          }
        }
        if (pn.j < it.m) load_state(chunk_at(it, pn));
      }
      p = pn;
      __syncthreads();  // chunk q + 1 is prepared
    }
    return;
  }

  // ---- producer waves.  While the state waves work on stream chunk q:
  //  waves 4 / 5: diagonal block 0 / 1 of T for chunk q + 2;
  //  wave 6: K tile and decay vectors of chunk q + 1, then A_10 and T_10 of
  //          chunk q + 1 (its diagonal blocks were solved one iteration earlier);
  //  wave 7: Q tile and P tiles of chunk q + 1, then its V tile once the
  //          state waves have released the V tile of chunk q.
  // Next-chunk loads go out right after the registers have been staged.
  // A prologue fills the pipeline: diagonal blocks of chunks 0 and 1 and
  // everything else of chunk 0.  Each role keeps its own stream positions.
  const int pw = wave - 4;
  if (pw < 2) {
    float* dgam = sm.dvec[pw][0];
    float* dbeta = sm.dvec[pw][1];
    float* deg = sm.dvec[pw][2];
    float* dieg = sm.dvec[pw][3];
    DiagLoad dl;
    Pos ps = first;  // the chunk whose loads are in dl
    auto dload = [&](Pos p) __attribute__((always_inline)) {
      const ChunkAt ch = chunk_at(it, p);
      load_diag(dl, source_of(a, ch), ch.c0, pw, lane, PAD ? a.kd : KD);
    };
    // solve this wave's diagonal block of stream chunk q (position ps) into T
    // buffer q % 3; the loads of the next chunk go out once the fragments are consumed
    auto solve = [&](int q) __attribute__((always_inline)) {
      float gl;
      const int L = chunk_at(it, ps).L;
      const float gm = chunk_gamma(dl.d, L, lane, gl);
      dgam[lane] = gm;
      deg[lane] = __expf(gm);
      dieg[lane] = __expf(-gm);
      const bool fact = factorable(gm);
      dbeta[lane] = lane < L ? scalar_raw_f32(dl.d.b, a.b_dtype) : 0.f;
      if constexpr (PAD) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
          if (16 * ks + 8 * (lane >> 5) >= a.kd) dl.kf[ks] = bf16x8{};
      }
      const f32x16 G = gram_regs<F16>(dl.kf);
      // max_i |k_i|^2 over this block's rows: the largest |k_i.k_j| of the Gram (Cauchy-Schwarz)
      {
        float m = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) m = fmaxf(m, fabsf(G[j]));
        m = wave_max(m);
        if (lane == 0) sm.kn2[q % 3][pw] = m;
      }
      ps = next_pos(it, ps);
      if (q + 1 < nq) dload(ps);
      solve_diag_block(sm.tb[q % 3], dgam, dbeta, deg, dieg, fact, G, pw, lane);
    };
    // Several items: the state waves load item j + 1's state right after
    // storing item j's.  These two waves touch it (one dword per 64 bytes,
    // half the state each) after their solve of the chunk before it, so that
    // the load finds most of it in L2.  Earlier touches lose more lines to
    // eviction before the load (measured: touching before the solve reads
    // 0.65 GB more from HBM on 512 x 64-token sequences, two chunks ahead is
    // slower still).  A touch's registers are folded into an accumulator one
    // touch later, so the wave never waits for one.
    Pos pp = first;  // stream chunk q + 1
    uint32_t pacc = 0, pv[8] = {};
    if constexpr (MULTI && !PAD)
      if (pp.j < it.m) pp = next_pos(it, pp);
    auto touch = [&]() __attribute__((always_inline)) {
      if (pp.j < it.m && pp.c == 0 && !(a.flags & GDN_PREFILL_ZERO_INIT)) {
        const ChunkAt ch = chunk_at(it, pp);
        const uint32_t* src = reinterpret_cast<const uint32_t*>(a.state + (int64_t)ch.slot * a.st_slot +
                                                                ch.h * a.st_head) + pw * (KD * VD / 2) + 16 * lane;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          pacc |= pv[i];
          pv[i] = src[1024 * i];
        }
      }
      if (pp.j < it.m) pp = next_pos(it, pp);
    };
    dload(ps);
    solve(0);
    producer_arrive(&sm.pro, lane);
    producer_wait(&sm.pro, 4, a.spin_limit, &sm.failed);
    if (nq > 1) solve(1);
    __syncthreads();
    for (int q = 0; q < nq; ++q) {
      if (q + 2 < nq) solve(q + 2);
      if constexpr (MULTI && !PAD) touch();
      __syncthreads();
    }
    if constexpr (MULTI && !PAD) {
#pragma unroll
      for (int i = 0; i < 8; ++i) pacc |= pv[i];
      asm volatile("" ::"v"(pacc));
    }
  } else if (pw == 2) {
    TileLoad kl;
    DecayLoad dl;
    Pos pl = first;  // the chunk whose loads are in kl / dl
    auto load = [&]() __attribute__((always_inline)) {
      const ChunkAt ch = chunk_at(it, pl);
      const ChunkSource src = source_of(a, ch);
      const int Lc = chunk_rows(src, ch.c0);
      load_tile(kl, src.kg, a.k_s0, ch.c0, Lc, lane, PAD ? a.kd : KD);
      load_decay(dl, src, ch.c0, Lc, lane);
    };
    // K tile and decay vectors of stream chunk q into tile set q & 1, then release wave 7
    auto stage = [&](int q) __attribute__((always_inline)) {
      ChunkTiles& ct = sm.tiles[q & 1];
      stage_f16<F16>(ct.k, kl, lane, !PAD || 8 * (lane & 15) < a.kd);
      stage_decay(ct, dl, chunk_at(it, pl).L, a.b_dtype, lane);
      producer_arrive(&sm.kv_ready, lane);
      pl = next_pos(it, pl);
    };
    auto offdiag = [&](int q) __attribute__((always_inline)) {
      b10_block(sm.tiles[q & 1], sm.tb[q % 3], lane);
      merge_offdiag(sm.tb[q % 3], lane);
    };
    load();
    stage(0);
    producer_arrive(&sm.pro, lane);
    producer_wait(&sm.pro, 4, a.spin_limit, &sm.failed);
    offdiag(0);
    if (nq > 1) load();
    __syncthreads();
    for (int q = 0; q < nq; ++q) {
      if (q + 1 < nq) {
        stage(q + 1);
        if (q + 2 < nq) load();
        offdiag(q + 1);
      }
      __syncthreads();
    }
  } else {
    TileLoad ql, vl;
    Pos pq = first, pv = first;  // the chunks whose loads are in ql / vl
    auto qload = [&]() __attribute__((always_inline)) {
      const ChunkAt ch = chunk_at(it, pq);
      const ChunkSource src = source_of(a, ch);
      load_tile(ql, src.qg, a.q_s0, ch.c0, chunk_rows(src, ch.c0), lane, PAD ? a.kd : KD);
    };
    auto vload = [&]() __attribute__((always_inline)) {
      const ChunkAt ch = chunk_at(it, pv);
      const ChunkSource src = source_of(a, ch);
      load_tile(vl, src.vg, a.v_s0, ch.c0, chunk_rows(src, ch.c0), lane, PAD ? a.vd : VD);
    };
    // Q tile and the three P tiles of stream chunk q
    auto qp = [&](int q) __attribute__((always_inline)) {
      ChunkTiles& ct = sm.tiles[q & 1];
      stage_f16<F16>(ct.q, ql, lane, !PAD || 8 * (lane & 15) < a.kd);
      pq = next_pos(it, pq);
      if (q + 1 < nq) qload();
      producer_wait(&sm.kv_ready, q + 1, a.spin_limit, &sm.failed);
      p_tile(ct, 0, 0, lane);
      p_tile(ct, 1, 0, lane);
      p_tile(ct, 1, 1, lane);
    };
    auto vstage = [&]() __attribute__((always_inline)) {
      stage_v(sm.v, vl, lane, !PAD || 8 * (lane & 15) < a.vd);
      pv = next_pos(it, pv);
    };
    qload();
    vload();
    qp(0);
    vstage();
    if (nq > 1) vload();
    producer_arrive(&sm.pro, lane);
    producer_wait(&sm.pro, 4, a.spin_limit, &sm.failed);
    __syncthreads();
    for (int q = 0; q < nq; ++q) {
      if (q + 1 < nq) {
        qp(q + 1);
        producer_wait(&sm.v_free, 4 * (q + 1), a.spin_limit, &sm.failed);  // the state waves are done with chunk q's V tile
        vstage();
        if (q + 2 < nq) vload();
      }
      __syncthreads();
    }
  }
}

GDN_DEVICE void reset_counters(Smem& sm) {
  sm.kv_ready = 0;
  sm.v_free = 0;
  sm.pro = 0;
  sm.failed = 0;
}

// MULTI: several items per workgroup (a.per_wg > 0), dealt by cost; the
// one-item schedule is its own instantiation, so the long-sequence path pays
// nothing for the item stream.
template <bool F16, bool MULTI, bool PAD, bool OUT32>
__global__ __launch_bounds__(kThreads) void gdn_chunk_prefill_kernel(PrefillArgs a) {
  __shared__ Smem sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int64_t bid = blockIdx.x;
  const int64_t nwork = a.nseq * a.Hv;

  if (!(a.flags & GDN_PREFILL_ACCUM_OUT))
    zero_uncovered_rows<OUT32 ? 4 : 2>(a.out, a.o_s0, a.o_s1, a.Hv, a.vd, a.cu, a.cu64, a.nseq, a.T, bid, gridDim.x,
                                       tid, kThreads);
  if constexpr (!MULTI) {
    // One item per workgroup: consecutive v-heads (sharing a k-head) go to one
    // XCD (workgroups are dealt round-robin over the 8 XCDs), sequences
    // longest first.
    const int64_t work = 2 * ((bid >> 4) * 8 + (bid & 7)) + ((bid >> 3) & 1);
    if (work >= nwork) return;
    if (tid == 0) reset_counters(sm);
    __syncthreads();  // the counters are zero before any wave can arrive
    Items it;
    it.m = 1;
    item_fields(a, seq_of_rank(sm, a, work / a.Hv, tid), (int)(work % a.Hv), it);
    run_items<F16, MULTI, PAD, OUT32>(sm, a, it, tid);
  } else {
    // A run of work ids, walked as streams of up to 64 items (one item per
    // lane of the item table); the v-head pairs of a k-head are consecutive
    // and share the workgroup's L2.
    int64_t w0, w1;
    multi_run(a, bid, gridDim.x, lane, w0, w1);
    for (int64_t base = w0; base < w1; base += 64) {
      // (an opaque thread index and an opaque pointer to the kernel
      // arguments per stream: nothing lane-dependent and no argument load is
      // hoisted out of this loop, where it would stay live across every
      // stream; the arguments are the kernel's only ones, at offset 0 of its
      // argument segment)
      int t = tid;
      asm volatile("" : "+v"(t));
#if defined(__HIP_DEVICE_COMPILE__)
      typedef const __attribute__((address_space(4))) PrefillArgs* KernArgs;
      KernArgs kp = (KernArgs)__builtin_amdgcn_kernarg_segment_ptr();
      asm volatile("" : "+s"(kp));
      const PrefillArgs as = *kp;  // (scalar loads from the constant address space)
#else
      const PrefillArgs& as = a;  // (the host pass only checks the kernel)
#endif
      if (t == 0) reset_counters(sm);
      __syncthreads();  // the counters are zero before any wave can arrive
      Items it;
      it.m = (int)(w1 - base < 64 ? w1 - base : 64);
      const int64_t w = base + ((t & 63) < it.m ? (t & 63) : 0);
      item_fields(as, w / as.Hv, (int)(w % as.Hv), it);
      run_items<F16, MULTI, PAD, OUT32>(sm, as, it, t);
      __syncthreads();  // every role has left the stream before the counters are reset
    }
  }
}

}  // namespace

// CUs of the device the stream runs on (the schedule heuristic's unit).
static int64_t stream_cu_count(hipStream_t st) {
  hipDevice_t dev = 0;
  int cus = 0;
  if (hipStreamGetDevice(st, &dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;  // (an MI355X; the result only shapes the schedule)
  return cus;
}

hipError_t gdn_chunk_prefill_launch(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v,
                                    const gdn_tensor* g, const gdn_tensor* beta, gdn_tensor* state,
                                    const gdn_tensor* idx, const gdn_tensor* cu, gdn_tensor* out, float scale,
                                    int32_t flags, int32_t spin_limit, int32_t items_per_wg, hipStream_t st) {
  PrefillArgs a;
  a.q = reinterpret_cast<const bf16_t*>(q->data);
  a.k = reinterpret_cast<const bf16_t*>(k->data);
  a.v = reinterpret_cast<const bf16_t*>(v->data);
  a.g = reinterpret_cast<const float*>(g->data);
  a.beta = beta->data;
  a.state = reinterpret_cast<float*>(state->data);
  a.idx = idx->data;
  a.cu = cu->data;
  a.out = reinterpret_cast<bf16_t*>(out->data);
  a.q_s0 = q->stride[0]; a.q_s1 = q->stride[1];
  a.k_s0 = k->stride[0]; a.k_s1 = k->stride[1];
  a.v_s0 = v->stride[0]; a.v_s1 = v->stride[1];
  a.g_s0 = g->stride[0]; a.g_s1 = g->stride[1];
  a.b_s0 = beta->stride[0]; a.b_s1 = beta->stride[1];
  a.o_s0 = out->stride[0]; a.o_s1 = out->stride[1];
  a.st_slot = state->stride[0]; a.st_head = state->stride[1];
  a.T = q->shape[0];
  a.nseq = cu->shape[0] - 1;
  a.num_slots = state->shape[0];
  a.Hv = (int32_t)v->shape[1];
  a.r = (int32_t)(v->shape[1] / q->shape[1]);
  a.b_dtype = beta->dtype;
  a.scale = scale;
  a.spin_limit = spin_limit;
  a.flags = flags;
  a.idx64 = idx->dtype == GDN_DTYPE_I64;
  a.cu64 = cu->dtype == GDN_DTYPE_I64;
  a.kd = (int32_t)q->shape[2];
  a.vd = (int32_t)v->shape[2];
  const int64_t nwork = a.nseq * a.Hv;
  if (a.T == 0) return hipSuccess;
  // Batches of short sequences (at most two chunks on average) with at least
  // two items per CU: each workgroup walks a run of about `per` items priced
  // by their tokens as one chunk stream, so that the next item's pipeline
  // fill overlaps the current item's chunks.  Otherwise one item per
  // workgroup, longest first.
  if (items_per_wg < 0) {
    const int64_t cus = stream_cu_count(st);
    const bool short_items = a.T <= 2 * C * a.nseq && nwork >= 2 * cus;
    const int64_t per = (nwork + cus - 1) / cus;
    items_per_wg = short_items ? (int32_t)(per < 64 ? per : 64) : 0;
  }
  a.per_wg = items_per_wg;
  // (with no items the launch still zeroes the rows no sequence covers)
  const int64_t nblocks = nwork == 0 ? 16
                          : items_per_wg > 0 ? (nwork + items_per_wg - 1) / items_per_wg
                                             : (nwork + 15) / 16 * 16;  // the work-id map covers whole groups of 16
  const dim3 grid((unsigned)nblocks), block(kThreads);
  const bool f16 = q->dtype == GDN_DTYPE_F16, multi = items_per_wg > 0, pad = a.kd != KD || a.vd != VD;
  const bool out32 = out->dtype == GDN_DTYPE_F32;  // (q, k, v fp16: checked by the caller)
#define GDN_PREFILL_LAUNCH(F16, MULTI, PAD, OUT32) \
  gdn_chunk_prefill_kernel<F16, MULTI, PAD, OUT32><<<grid, block, 0, st>>>(a)
#define GDN_PREFILL_BY_PAD(F16, MULTI, OUT32)                   \
  do {                                                           \
    if (pad) GDN_PREFILL_LAUNCH(F16, MULTI, true, OUT32);        \
    else GDN_PREFILL_LAUNCH(F16, MULTI, false, OUT32);           \
  } while (0)
#define GDN_PREFILL_BY_MULTI(F16, OUT32)                         \
  do {                                                           \
    if (multi) GDN_PREFILL_BY_PAD(F16, true, OUT32);             \
    else GDN_PREFILL_BY_PAD(F16, false, OUT32);                  \
  } while (0)
  if (out32) GDN_PREFILL_BY_MULTI(true, true);
  else if (f16) GDN_PREFILL_BY_MULTI(true, false);
  else GDN_PREFILL_BY_MULTI(false, false);
#undef GDN_PREFILL_BY_MULTI
#undef GDN_PREFILL_BY_PAD
#undef GDN_PREFILL_LAUNCH
  return hipGetLastError();
}
