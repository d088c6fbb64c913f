// Full-attention kernels of the hybrid stack for gfx950: varlen and paged
// prefill on 32x32x16 MFMA tiles, split-KV paged decode on 16x16 tiles.
//
// Reference: ops/full_attention.py of yuyifanbupt/myvllm (flash_attention_prefill
// :114-173, paged_flash_attention_decode :282-335, paged_flash_attention_prefill
// :454-512).  Query head h reads kv head h / (Hq / Hkv); softmax in fp32 with a
// running maximum; P rounded to the input dtype before P V, the row sum taken
// over the unrounded fp32 P (:100-107).
//
// Layout of the prefill tile: the score tile is computed transposed,
// S^T = K Q^T, so that lane l of a wave owns query column l % 32 of the
// accumulator.  The softmax statistics of a query then live in one lane pair
// (l, l ^ 32), and the exponentiated accumulator registers are already the B
// operand of O^T = V^T P^T, whose A operand is read from the row-major V tile
// with ds_read_b64_tr_b16.  The running maximum is re-based only when a new
// tile raises it by more than 2^8 (in exp2 units); O and the row sum always
// share the same base, so the result is the same softmax.
#include "gdn_common.h"

#include <mutex>

// Split partials of paged_attention_decode_noalloc: a file-scope device array
// (one copy per GPU, for the life of the process) instead of a caller
// workspace.  Host code never passes `scratch` itself to a kernel (on the host
// the name stands for a host-side shadow, not a device address): the address
// is looked up once per device with hipGetSymbolAddress.
static __device__ __align__(256) float scratch[GDN_DECODE_SCRATCH_FLOATS];

namespace {

template <typename T> struct Mma;
template <> struct Mma<bf16_t> {
  typedef bf16x8 v8;
  typedef bf16x4 v4;
  static GDN_DEVICE f32x16 m32(v8 a, v8 b, f32x16 c) { return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0); }
  static GDN_DEVICE f32x4 m16k32(v8 a, v8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
  static GDN_DEVICE f32x4 m16k16(v4 a, v4 b, f32x4 c) {
    typedef short s4 __attribute__((ext_vector_type(4)));
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4, a), __builtin_bit_cast(s4, b), c, 0, 0, 0);
  }
};
template <> struct Mma<f16_t> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef _Float16 v4 __attribute__((ext_vector_type(4)));
  static GDN_DEVICE f32x16 m32(v8 a, v8 b, f32x16 c) { return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0); }
  static GDN_DEVICE f32x4 m16k32(v8 a, v8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
  static GDN_DEVICE f32x4 m16k16(v4 a, v4 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }
};

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef short __attribute__((address_space(3))) lds_short;
typedef s16x4_t __attribute__((address_space(3))) lds_s16x4_t;

// ds_read_b64_tr_b16: in each 16-lane group, lane i supplies the address of
// 4 consecutive 16-bit elements of row (i >> 2), columns 4 (i & 3) .. +3, of
// a 4 x 16 block, and receives column i of that block (rows 0..3).
template <typename V4> GDN_DEVICE V4 tr4(const void* p) {
  return __builtin_bit_cast(V4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p)));
}

GDN_DEVICE float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// max(x[l], x[l ^ 32]) in every lane l: one v_permlane32_swap of x with
// itself (lanes 0..31 of one copy trade places with lanes 32..63 of the
// other, so each lane then holds both of the pair's values), no LDS round
// trip as a ds_bpermute would take.  (The two results are copied to scalars
// before they are reinterpreted: this clang reads the first element of the
// vector for __builtin_bit_cast(float, sw[1]).)  The maximum is a select:
// fmaxf would first quiet both operands, two more instructions on the
// softmax's dependency chain (the scores are never NaN).
GDN_DEVICE float max_lane_pair32(float x) {
  const uint32_t v = __builtin_bit_cast(uint32_t, x);
  const auto sw = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  const uint32_t ua = sw[0], ub = sw[1];
  const float a = __builtin_bit_cast(float, ua), b = __builtin_bit_cast(float, ub);
  return a > b ? a : b;
}

GDN_DEVICE int64_t clamp64(int64_t x, int64_t lo, int64_t hi) { return x < lo ? lo : (x > hi ? hi : x); }

// An index at a wave-uniform position read through the scalar data cache (a
// constant-address-space load): its wait is on the scalar/LDS counter, so it
// does not drain the vector loads in flight.  Only for read-only inputs.
typedef const int32_t __attribute__((address_space(4))) * const_i32_ptr;
typedef const int64_t __attribute__((address_space(4))) * const_i64_ptr;
GDN_DEVICE int64_t load_index_scalar(const void* p, int64_t i, bool is64) {
  return is64 ? __builtin_bit_cast(const_i64_ptr, p)[i] : (int64_t)__builtin_bit_cast(const_i32_ptr, p)[i];
}

// Row j of a key or value source: packed varlen rows (row s0 + j) or paged
// rows (block table[n][j / page], slot j % page).  nullptr past the valid
// range or for a table entry outside [0, num_blocks): such rows read as zero.
struct KvSource {
  const char* base;
  int64_t sb, st, sh;  // byte strides: block (paged), row, head
};

struct PagedTable {
  const void* table;
  int64_t row_stride, cols, num_blocks;
  int32_t page;
  bool is64;
};

struct AttnArgs {
  const void* q;
  int64_t q_st, q_sh;  // element strides: token, head
  KvSource k, v;
  void* o;
  int64_t o_st, o_sh;
  const void* cu;
  const void* ctx;
  PagedTable tab;
  int64_t T, nseq;
  int32_t Hq, Hkv, gh;  // gh: query heads per workgroup (1, 2 or 4)
  float c;              // softmax scale * log2(e)
  bool cu64, ctx64, causal;
};

template <bool PAGED>
GDN_DEVICE const char* kv_row(const KvSource& s, const PagedTable& tb, int64_t n, int64_t s0, int64_t j, int kvh) {
  if (PAGED) {
    const int64_t col = j / tb.page;
    if (col >= tb.cols) return nullptr;
    const int64_t blk = load_index(tb.table, n * tb.row_stride + col, tb.is64);
    if (blk < 0 || blk >= tb.num_blocks) return nullptr;
    return s.base + blk * s.sb + (j - col * tb.page) * s.st + kvh * s.sh;
  } else {
    return s.base + (s0 + j) * s.st + kvh * s.sh;
  }
}

// ---------------------------------------------------------------------------
// Prefill: one workgroup = 4 waves = `gh` query heads of one kv head x
// (4 / gh) blocks of 32 queries.  K and V tiles of BN keys are staged in LDS
// (double buffered, the next tile prefetched into registers) and shared by
// the four waves.
// PG: 0 packed rows, 1 paged (any page size: a table lookup per row),
// 2 / 3 paged with a page size that is a multiple of 16 and an int32 / int64
// block table (one lookup per 16 rows, a tile ahead, 32-bit arithmetic)
// Workgroup id -> (sequence, query tile): tiles of tile_len queries, laid out
// sequence after sequence over the tiles that exist (no workgroup of a
// padded grid exits idle).  Out of line, so that the lookup's registers and
// barriers leave the kernel's own allocation alone.
struct SeqTile {
  int64_t seq, tile;
};
__device__ __attribute__((always_inline)) SeqTile attn_tile_lookup(const void* cu, bool cu64, int64_t nseq, int64_t T,
                                                              int tile_len, int64_t target, int32_t* lds) {
  SeqTile r;
  find_seq_tile<256>(cu, cu64, nseq, T, tile_len, target, r.seq, r.tile, lds);
  return r;
}

template <typename T, int D, int BN, int PG>
__global__ __launch_bounds__(256) void attn_prefill_kernel(const AttnArgs a) {
  constexpr bool PAGED = PG != 0;
  typedef Mma<T> M;
  typedef typename M::v8 v8;
  typedef typename M::v4 v4;
  constexpr int LDK = D + 8;   // row stride (elements): 16-byte row skew for the b128 reads
  constexpr int LDV = D + 32;  // 64-byte row skew for the transposed reads
  constexpr int NKS = D / 16;
  constexpr int NA = BN / 32;
  constexpr int NDT = D / 32;
  constexpr int CH = D / 8;  // 16-byte chunks per row
  constexpr int NLD = BN * CH / 256;
  static_assert(BN % 32 == 0 && (BN * CH) % 256 == 0, "tile");
  __shared__ __align__(16) T ks[2][BN * LDK];
  __shared__ __align__(16) T vs[2][BN * LDV];
  // D = 256: each wave's query fragments sit in LDS (16.5 KB per wave)
  // instead of 64 VGPRs; the registers this frees hold the K, Q and V
  // fragments of the next MFMAs while the current one runs (with Q resident
  // the allocator kept one fragment buffer, so every LDS read was waited for
  // right before its MFMA)
  constexpr bool QL = D == 256;
  // of those, the last QRG stay in registers as well (fewer LDS reads in the
  // score phase for 48 more registers; measured: 12 of 16, all 16 much slower)
  constexpr int QRG = QL ? 12 : 0;
  __shared__ __align__(16) T qs[QL ? 4 * 32 * LDK : 8];

  // (the wave index through readfirstlane: the compiler then knows it, and
  // the wave's query block, causal range and tile tests, to be uniform, so
  // they live in scalar registers and branch without exec masks)
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int R = a.Hq / a.Hkv, gh = a.gh, qsubs = 4 / gh, groups = R / gh;
  // Workgroup order: sequence after sequence, a sequence's query tiles last
  // first, the head groups of a tile innermost.  The dispatcher deals
  // consecutive workgroups to its 32 queues (8 XCDs x 4 shader engines, 8
  // CUs each) in turn, so every sequence spreads over all of them, and a
  // sequence's workgroups run together and share its K/V rows in L2.
  __shared__ int32_t lookup[8];
  const int hg = a.Hq / gh;  // head groups
  const SeqTile st = attn_tile_lookup(a.cu, a.cu64, a.nseq, a.T, 32 * qsubs, blockIdx.x / hg, lookup);
  if (st.seq < 0) return;
  const int64_t n = st.seq;
  const int y = (int)(blockIdx.x % hg);
  const int kvh = y / groups;
  const int head = kvh * R + (y % groups) * gh + (w % gh);

  int64_t s0, s1;
  seq_range(a.cu, a.cu64, n, a.T, s0, s1);
  const int64_t len = s1 - s0;
  const int64_t ntile = (len + 32 * qsubs - 1) / (32 * qsubs);
  const int64_t qb = (ntile - 1 - st.tile) * 32 * qsubs;  // last query tiles first

  int64_t Lk, off;
  if (PAGED) {
    const int64_t ctx = load_index(a.ctx, n, a.ctx64);
    Lk = clamp64(ctx, 0, a.tab.cols * a.tab.page);
    off = ctx - len;  // position of query 0
  } else {
    Lk = len;
    off = 0;
  }
  const int64_t q0 = qb + (w / gh) * 32;
  const int64_t wg_qend = qb + 32 * qsubs < len ? qb + 32 * qsubs : len;
  const int64_t w_qend = q0 + 32 < len ? q0 + 32 : len;
  const int64_t kend = a.causal ? clamp64(off + wg_qend, 0, Lk) : Lk;
  const int64_t kend_w = q0 >= len ? 0 : (a.causal ? clamp64(off + w_qend, 0, Lk) : Lk);
  const int ntiles = (int)((kend + BN - 1) / BN);

  // query fragments (B operand of S^T = K Q^T): lane holds query q0 + lane % 32,
  // dims 16 ks + 8 (lane / 32) .. +7
  const int col = lane & 31, hh = lane >> 5;
  const int64_t qi = q0 + col;
  const bool qvalid = qi < len;
  // (loaded unconditionally from a clamped row, so the loads stay in flight
  // while tile 0's K/V loads are issued; rows past the sequence are zeroed
  // where the fragments are staged, below)
  v8 qf[NKS];
  {
    const T* qp = reinterpret_cast<const T*>(a.q) + (s0 + (qvalid ? qi : 0)) * a.q_st + (int64_t)head * a.q_sh + 8 * hh;
#pragma unroll
    for (int s = 0; s < NKS; ++s) qf[s] = *reinterpret_cast<const v8*>(qp + 16 * s);
  }
  // the softmax below assumes c > 0: a negative scale is folded into q (an
  // exact sign flip), a zero scale is q = 0 with c = 1 (equal weights)
  float c = a.c;
  T* const qw = qs + (QL ? w * 32 * LDK : 0);  // this wave's query rows (only the wave reads them)
  auto stage_q = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < NKS; ++s) qf[s] = qvalid ? qf[s] : v8{};
    if (c <= 0.f) {
#pragma unroll
      for (int s = 0; s < NKS; ++s) qf[s] = c < 0.f ? -qf[s] : v8{};
      c = c < 0.f ? -c : 1.f;
    }
    if constexpr (QL) {
#pragma unroll
      for (int s = 0; s < NKS - QRG; ++s) *reinterpret_cast<v8*>(qw + col * LDK + 16 * s + 8 * hh) = qf[s];
    }
  };

  // staging of a K/V tile: global rows -> registers (rows past kend read as
  // zero, so a tile past the range loads nothing) -> LDS
  // packed rows: per key tile, buffer descriptors of the tile's rows of this
  // sequence's kv head whose range ends at the last row before kend (rows
  // past it read as zero, 32-bit offsets): a lane's offsets are the same for
  // every tile, and the tile's position and bound are scalar arithmetic
  const char* const kseq = a.k.base + s0 * a.k.st + kvh * a.k.sh;
  const char* const vseq = a.v.base + s0 * a.v.st + kvh * a.v.sh;
  constexpr int NG = BN / 16;  // 16-row groups of a tile
  static_assert(CH >= 8 && 64 % CH == 0, "a wave's rows of a tile lie in one 16-row group");
  // PG 2, 3: each 16-row group of a tile lies in one page.  Its block id is a
  // vector load issued one tile ahead, before the previous tile's data loads,
  // so waiting for it leaves those data loads in flight (a scalar load would
  // be waited for at once, its value forming the addresses, and that wait
  // also drains every LDS access in flight).  The rows then load through a
  // buffer descriptor of the kv head's rows of the page: 32-bit offsets, rows
  // past the range or of an invalid block read zero.
  // The 16-row groups are enumerated in order (load_ids runs for tiles 0, 1,
  // 2, ...), so a group's table column and first page slot are counted up,
  // not divided out.
  // An id is kept as the two raw 32-bit words it was loaded as (an int32
  // table: the entry twice) and decoded only where it is used: converting it
  // at the load would wait for the load, and with it for every load in flight.
  uint32_t idlo[NG], idhi[NG];  // raw block ids of the next tile to load
  bool idin[NG];                // its groups lie inside the range and the table
  uint32_t slots[NG];           // their first page slot
  constexpr bool G16 = PG >= 2, T64 = PG == 3;  // 16-row groups per page lookup; int64 table
  const uint32_t gpp = G16 ? (uint32_t)a.tab.page / 16 : 1u;  // 16-row groups per page
  uint32_t gcol = 0, grem = 0;  // table column and group within the page of the next group
  // (G16) this sequence's row of the block table as 32-bit words; the table
  // has columns, and key positions (columns x page), block ids and block
  // strides fit 32 bits (the launcher takes the per-row path otherwise)
  const uint32_t* trow = G16 ? reinterpret_cast<const uint32_t*>(a.tab.table) + (T64 ? 2 : 1) * (n * a.tab.row_stride)
                             : nullptr;
  const uint32_t kend32 = (uint32_t)kend;
  auto load_ids = [&](int t, uint32_t* lo, uint32_t* hi, bool* in, uint32_t* sl) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const uint32_t j0 = (uint32_t)t * BN + 16 * g;
      in[g] = j0 < kend32 && gcol < a.tab.cols;
      // (the index goes through a vector register so the loads stay vector loads)
      uint32_t e = in[g] ? gcol : 0u;
      asm volatile("" : "+v"(e));
      if constexpr (T64) {
        lo[g] = trow[2 * e];
        hi[g] = trow[2 * e + 1];
      } else {
        lo[g] = trow[e];
        hi[g] = 0u;
      }
      sl[g] = 16 * grem;
      if (++grem == gpp) {
        grem = 0;
        ++gcol;
      }
    }
  };
  if (G16) load_ids(0, idlo, idhi, idin, slots);
  const uint32_t kst = (uint32_t)a.k.st, vst = (uint32_t)a.v.st;  // row strides in bytes (below 2^31)
  const char* kbase = a.k.base + kvh * a.k.sh;
  const char* vbase = a.v.base + kvh * a.v.sh;
  const uint64_t ksb = (uint32_t)a.k.sb, vsb = (uint32_t)a.v.sb;
  const uint32_t nblk = (uint32_t)(a.tab.num_blocks < 0x7fffffff ? a.tab.num_blocks : 0x7fffffff);
  auto load_tile = [&](int t, uint4* kd, uint4* vd) {
    __amdgpu_buffer_rsrc_t rkg[NG], rvg[NG], rkt, rvt;
    uint32_t r0[NG];
    if (!PAGED) {
      const uint32_t t0 = (uint32_t)t * BN;
      const uint32_t nv = t0 < kend32 ? (kend32 - t0 < (uint32_t)BN ? kend32 - t0 : (uint32_t)BN) : 0u;
      rkt = __builtin_amdgcn_make_buffer_rsrc((void*)(kseq + (uint64_t)t0 * kst), 0, nv * kst, 0x00020000);
      rvt = __builtin_amdgcn_make_buffer_rsrc((void*)(vseq + (uint64_t)t0 * vst), 0, nv * vst, 0x00020000);
    }
    if (G16) {
      uint32_t nlo[NG], nhi[NG], nsl[NG];
      bool nin[NG];
      load_ids(t + 1, nlo, nhi, nin, nsl);
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        // valid: inside the range, high word zero (int64) or non-negative (int32), below num_blocks
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int32_t)idlo[g]);
        const uint32_t hi = T64 ? (uint32_t)__builtin_amdgcn_readfirstlane((int32_t)idhi[g]) : 0u;
        // (an int32 id below nblk is non-negative: negative ids compare above it unsigned)
        const bool valid = idin[g] && hi == 0u && lo < nblk;
        const uint64_t bb = valid ? lo : 0u;
        r0[g] = slots[g];
        // the group's rows before kend: its range ends after them in the page,
        // so the rows past kend read as zero with no test per row
        const uint32_t j0 = (uint32_t)t * BN + 16u * g;
        const uint32_t ends = slots[g] + (j0 < kend32 ? (kend32 - j0 < 16u ? kend32 - j0 : 16u) : 0u);
        // (block strides below 2^32, checked by the launcher: 32 x 32-bit products)
        rkg[g] = __builtin_amdgcn_make_buffer_rsrc((void*)(kbase + bb * ksb), 0, valid ? ends * kst : 0u, 0x00020000);
        rvg[g] = __builtin_amdgcn_make_buffer_rsrc((void*)(vbase + bb * vsb), 0, valid ? ends * vst : 0u, 0x00020000);
        idlo[g] = nlo[g];
        idhi[g] = nhi[g];
        idin[g] = nin[g];
        slots[g] = nsl[g];
      }
    }
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int c = tid + 256 * i, row = c / CH, ch = c % CH;
      const int64_t j = (int64_t)t * BN + row;
      if (G16) {
        // the row's 16-row group: i * rows-per-pass / 16 when a pass covers at
        // most 16 rows (a constant), else plus the wave's part (uniform)
        constexpr int RPI = 256 / CH;
        __amdgpu_buffer_rsrc_t rkx, rvx;
        uint32_t rx;
        if constexpr (RPI <= 16) {
          rkx = rkg[i * RPI / 16];
          rvx = rvg[i * RPI / 16];
          rx = r0[i * RPI / 16];
        } else {
          const int gu = __builtin_amdgcn_readfirstlane(row >> 4);
          rkx = rkg[0], rvx = rvg[0], rx = r0[0];
#pragma unroll
          for (int g = 1; g < NG; ++g) {
            rkx = gu == g ? rkg[g] : rkx;
            rvx = gu == g ? rvg[g] : rvx;
            rx = gu == g ? r0[g] : rx;
          }
        }
        const uint32_t slot = rx + (uint32_t)(row & 15);
        kd[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rkx, slot * kst + 16u * ch, 0, 0));
        vd[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rvx, slot * vst + 16u * ch, 0, 0));
        continue;
      }
      if (!PAGED) {
        // (the row offset times the stride fits 32 bits: the launcher checks
        // max(max_seqlen, 64) rows of either stride against 2^31)
        kd[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rkt, (uint32_t)row * kst + 16u * ch, 0, 0));
        vd[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rvt, (uint32_t)row * vst + 16u * ch, 0, 0));
        continue;
      }
      const char* pk = j < kend ? kv_row<PAGED>(a.k, a.tab, n, s0, j, kvh) : nullptr;
      const char* pv = j < kend ? kv_row<PAGED>(a.v, a.tab, n, s0, j, kvh) : nullptr;
      kd[i] = pk ? *reinterpret_cast<const uint4*>(pk + 16 * ch) : uint4{0, 0, 0, 0};
      vd[i] = pv ? *reinterpret_cast<const uint4*>(pv + 16 * ch) : uint4{0, 0, 0, 0};
    }
  };
  auto store_tile = [&](int buf, const uint4* kd, const uint4* vd) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int c = tid + 256 * i, row = c / CH, ch = c % CH;
      *reinterpret_cast<uint4*>(&ks[buf][row * LDK + 8 * ch]) = kd[i];
      *reinterpret_cast<uint4*>(&vs[buf][row * LDV + 8 * ch]) = vd[i];
    }
  };

  f32x16 oacc[NDT];
#pragma unroll
  for (int d = 0; d < NDT; ++d) oacc[d] = f32x16{};
  float m_used = -INFINITY, lsum = 0.f;
  float nb = 0.f;  // -m_used, or 0 while m_used is -inf (the exponent offset)

  // a key tile needs the mask when it reaches past the keys (t BN + BN > Lk)
  // or, causal, past the wave's first query (t BN + BN - 1 > off + q0):
  // t BN > mthr, one 32-bit test per tile (key positions stay below 2^31)
  const int mthr = (int)clamp64(a.causal ? (Lk - BN < off + q0 - BN + 1 ? Lk - BN : off + q0 - BN + 1) : Lk - BN, -1,
                                0x7fffffff);
  // `mid` (the next tiles' LDS stores and global loads) is issued right after
  // the score MFMAs, so that its issue overlaps their execution; a wave with
  // no keys left in this tile still runs it
  auto compute = [&](int t, int buf, auto&& mid) {
    if ((int64_t)t * BN < kend_w) {
      const T* K = ks[buf];
      const T* V = vs[buf];
      f32x16 s[NA];
#pragma unroll
      for (int aa = 0; aa < NA; ++aa) {
        s[aa] = f32x16{};
        const T* kp = K + (32 * aa + col) * LDK + 8 * hh;
        if constexpr (QL) {
          const T* qp = qw + col * LDK + 8 * hh;
#pragma unroll
          for (int k = 0; k < NKS; ++k)
            s[aa] = M::m32(*reinterpret_cast<const v8*>(kp + 16 * k),
                           k >= NKS - QRG ? qf[k] : *reinterpret_cast<const v8*>(qp + 16 * k), s[aa]);
          // schedule: the K and Q fragments of the next k-steps are read while each MFMA runs
          __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // DS reads
#pragma unroll
          for (int k = 0; k < NKS; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            if (k + 2 < NKS - QRG) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            else if (k + 2 < NKS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
        } else {
#pragma unroll
          for (int k = 0; k < NKS; ++k) s[aa] = M::m32(*reinterpret_cast<const v8*>(kp + 16 * k), qf[k], s[aa]);
        }
      }
      mid();
      // mask keys past the sequence / context and, if causal, past the query
      const int64_t tk0 = (int64_t)t * BN;
      if (t * BN > mthr) {
        const int64_t lim = (a.causal ? (off + qi + 1 < Lk ? off + qi + 1 : Lk) : Lk) - tk0;
        const int rel = (int)clamp64(lim, -1, BN);  // keys of the tile at or past rel are masked
#pragma unroll
        for (int aa = 0; aa < NA; ++aa)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (32 * aa + 8 * (r >> 2) + 4 * hh + (r & 3) >= rel) s[aa][r] = -INFINITY;
      }
      // tile maximum of the scaled scores (c > 0) over this lane's half of
      // the query's keys; masked scores are -inf and give p = exp2(-inf) = 0
      // below.  The lane pair (l, l ^ 32) shares one base: it moves only when
      // some lane's half exceeds it by 2^8, and then to the maximum over the
      // pair, so the pair's maximum is taken only on that rare path (the
      // same decisions and bases as taking it every tile)
      float mx = -INFINITY;
#pragma unroll
      for (int aa = 0; aa < NA; ++aa)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[aa][r]);
      if (__builtin_amdgcn_ballot_w64(mx * c > m_used + 8.f) != 0) {
        const float mn = fmaxf(m_used, max_lane_pair32(mx) * c);
        const float alpha = mn == -INFINITY ? 1.f : exp2_fast(m_used - mn);
#pragma unroll
        for (int d = 0; d < NDT; ++d) oacc[d] *= alpha;
        lsum *= alpha;
        m_used = mn;
        nb = mn == -INFINITY ? 0.f : -mn;
      }
#pragma unroll
      for (int aa = 0; aa < NA; ++aa) {
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          v8 pf;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float p = exp2_fast(__builtin_fmaf(s[aa][8 * h2 + e], c, nb));
            lsum += p;
            pf[e] = (T)p;
          }
          // V^T fragment for keys 32 aa + 16 h2 + {4 hh + 0..3, 8 + 4 hh + 0..3}
          const int j16 = lane & 15, qd = lane >> 4;
          const T* vp = V + (32 * aa + 16 * h2 + 4 * (qd >> 1) + (j16 >> 2)) * LDV + 16 * (qd & 1) + 4 * (j16 & 3);
          auto vfrag = [&](int d) __attribute__((always_inline)) {
            const v4 lo = tr4<v4>(vp + 32 * d);
            const v4 hi = tr4<v4>(vp + 32 * d + 8 * LDV);
            return v8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          };
          if constexpr (QL) {
            // the V fragments of two MFMAs ahead are in flight while each
            // MFMA runs; the scheduling barrier keeps the reads ahead
            constexpr int AH = 2;
            v8 vf[AH + 1];
#pragma unroll
            for (int i = 0; i < AH; ++i) vf[i] = vfrag(i);
#pragma unroll
            for (int d = 0; d < NDT; ++d) {
              if (d + AH < NDT) vf[(d + AH) % (AH + 1)] = vfrag(d + AH);
              __builtin_amdgcn_sched_barrier(0);
              oacc[d] = M::m32(vf[d % (AH + 1)], pf, oacc[d]);
            }
          } else {
#pragma unroll
            for (int d = 0; d < NDT; ++d) oacc[d] = M::m32(vfrag(d), pf, oacc[d]);
          }
        }
      }
    } else {
      mid();
    }
  };

  // tile t computes from LDS buffer t % 2 while tile t + 1 waits in registers
  // and tile t + 2 is in flight: two register sets (A: even tiles, B: odd)
  uint4 kA[NLD], vA[NLD], kB[NLD], vB[NLD];
  load_tile(0, kA, vA);
  stage_q();  // (waits for the query loads with tile 0's loads in flight)
  store_tile(0, kA, vA);
  load_tile(1, kB, vB);
  load_tile(2, kA, vA);
  __syncthreads();
  // (packed rows: the next tiles' stores and loads go out between the score
  // MFMAs and the softmax; paged rows: after the tile, since their loads
  // first wait for the block ids, and the longer live ranges cost registers)
  for (int t = 0; t < ntiles; t += 2) {
    if constexpr (PG == 0) {
      compute(t, 0, [&]() __attribute__((always_inline)) {
        store_tile(1, kB, vB);
        load_tile(t + 3, kB, vB);
      });
      __syncthreads();
      compute(t + 1, 1, [&]() __attribute__((always_inline)) {
        store_tile(0, kA, vA);
        load_tile(t + 4, kA, vA);
      });
      __syncthreads();
    } else {
      const auto after = []() {};  // (one instantiation of compute for both calls)
      compute(t, 0, after);
      store_tile(1, kB, vB);
      load_tile(t + 3, kB, vB);
      __syncthreads();
      compute(t + 1, 1, after);
      store_tile(0, kA, vA);
      load_tile(t + 4, kA, vA);
      __syncthreads();
    }
  }

  const float lt = lsum + __shfl_xor(lsum, 32);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  if constexpr (QL) {
    // O goes out through the wave's own query rows in LDS (no longer read):
    // each lane writes its 4-dim pieces of its query's row, then reads back
    // 16-byte row pieces, so that one store instruction covers two whole
    // output rows (512 contiguous bytes each) instead of 32 rows x 16 bytes
#pragma unroll
    for (int d = 0; d < NDT; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        v4 ov;
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = (T)(oacc[d][4 * g + e] * inv);
        *reinterpret_cast<v4*>(qw + col * LDK + 32 * d + 8 * g + 4 * hh) = ov;
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int cpos = lane & (CH - 1), rsub = lane / CH;  // 16-byte piece of a row, row within the pass
    constexpr int RPP = 64 / CH;                           // rows per pass
    const int qrem = (int)clamp64(len - q0, 0, 32);  // rows of this wave inside the sequence
    T* const orow = reinterpret_cast<T*>(a.o) + (s0 + q0) * a.o_st + (int64_t)head * a.o_sh + 8 * cpos;
#pragma unroll
    for (int r0 = 0; r0 < 32; r0 += RPP) {
      const int r = r0 + rsub;
      const v8 ov = *reinterpret_cast<const v8*>(qw + r * LDK + 8 * cpos);
      if (r < qrem) *reinterpret_cast<v8*>(orow + (int64_t)r * a.o_st) = ov;
    }
  } else if (qvalid) {
    T* op = reinterpret_cast<T*>(a.o) + (s0 + qi) * a.o_st + (int64_t)head * a.o_sh + 4 * hh;
#pragma unroll
    for (int d = 0; d < NDT; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        v4 ov;
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = (T)(oacc[d][4 * g + e] * inv);
        *reinterpret_cast<v4*>(op + 32 * d + 8 * g) = ov;
      }
  }
}

// ---------------------------------------------------------------------------
// Paged decode: one wave per (kv head, group of up to 16 query heads) of a
// work unit.  The query heads of one kv head are the 16 columns of
// S^T = K Q^T (16x16x32 MFMA, K fragments straight from global memory), the
// V tile goes through a wave-private LDS tile for the transposed read of
// O^T = V^T P^T (16x16x16 MFMA).  With one split a unit is one sequence and
// the wave writes the normalised output.  With num_splits > 1 the batch is
// dealt evenly over U = B (num_splits - 1) units by price: sequence b costs
// its 16-key tiles T_b = ceil(L_b / 16) plus kDecodeStartPrice for the start
// of a piece (its query load and pipeline fill), 0 if it has no keys; laid
// end to end the sequences fill prices [0, Q_B), sequence b's tiles at
// [Q_b + kDecodeStartPrice, Q_{b+1}), and unit u takes the tiles whose prices
// lie in [u Q_B / U, (u+1) Q_B / U).  So every unit streams about the same
// number of keys whatever the lengths are.  A unit crossing sequence ends
// runs one piece per sequence.  A piece that is a whole sequence writes its
// output row; any other piece (sequence b, unit u) writes its unnormalised O,
// running maximum and row sum to workspace slot b + u < B + U (distinct for
// distinct pieces: a later piece has a later unit or a later sequence and
// neither index decreases), which attn_decode_combine_kernel merges.  The
// price prefix Q is summed by the decode waves themselves for batches of up to
// 1,024 sequences, else by attn_decode_prices_kernel, launched first.  With a
// page size that is a multiple of 16 a 16-key tile lies in one page: its block
// id is one wave-uniform load, issued a tile ahead of the K/V loads that use
// it.  The kvw kv heads of a workgroup (one wave
// each) read the interleaved head rows of the same cache slots at about the
// same time, so each page is streamed as one contiguous region.
constexpr int32_t kDecodeStartPrice = 2;

struct DecodeArgs {
  const void* q;
  int64_t q_ss, q_sh;
  KvSource k, v;
  void* o;
  int64_t o_ss, o_sh;
  const void* ctx;
  PagedTable tab;
  float* part;     // (B + U = B splits, Hq, D + 4): O, m, l per piece (rows padded to 16 bytes)
  int32_t* prices;  // (B + 1): the price prefix Q (splits > 1)
  int32_t B, Hq, Hkv, splits, kvw;
  int32_t units;  // splits > 1: units per sequence, splits - 1 (U = B units)
  float c;
  bool ctx64;
  bool prices_inline;  // the decode waves compute Q themselves (small batches)
};

// Price prefix of the batch for the split decode: Q[b] = sum over b' < b of
// the price of b' (ceil(L_b' / 16) + kDecodeStartPrice, or 0 with no keys),
// Q[B] the total, with L_b the context length clamped to the table's capacity
// as the decode clamps it.  One workgroup: each thread sums a contiguous run of
// sequences, the run sums are scanned across the block, and each thread writes
// its run's prefixes.  (Q[B] < 2^31: the entry point checks
// B * (ceil(capacity / 16) + kDecodeStartPrice).)
__global__ __launch_bounds__(1024) void attn_decode_prices_kernel(const DecodeArgs a) {
  __shared__ int32_t wsum[16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t cap = a.tab.cols * a.tab.page;
  const int per = (a.B + 1023) / 1024;
  const int64_t b0 = (int64_t)tid * per;
  auto price_of = [&](int64_t b) -> int32_t {
    const int32_t t = b < a.B ? (int32_t)((clamp64(load_index(a.ctx, b, a.ctx64), 0, cap) + 15) / 16) : 0;
    return t > 0 ? t + kDecodeStartPrice : 0;
  };
  int32_t sum = 0;
  for (int i = 0; i < per; ++i) sum += price_of(b0 + i);
  // inclusive scan over the wave, then over the 16 wave totals
  int32_t inc = sum;
#pragma unroll
  for (int d = 1; d < 64; d *= 2) {
    const int32_t y = __shfl_up(inc, d);
    if (lane >= d) inc += y;
  }
  if (lane == 63) wsum[w] = inc;
  __syncthreads();
  int32_t base = 0;
  for (int i = 0; i < w; ++i) base += wsum[i];
  int32_t run = base + inc - sum;  // exclusive prefix of this thread's run
  for (int i = 0; i < per; ++i) {
    const int64_t b = b0 + i;
    if (b >= a.B) break;
    a.prices[b] = run;
    run += price_of(b);
  }
  if (tid == 1023) a.prices[a.B] = base + inc;
}

// LDS bytes of one decode wave: a 16-row V tile with a 32-byte row skew and
// the wave's query fragments
template <typename T, int D>
constexpr size_t decode_lds_per_wave() { return (size_t)16 * (D + 16) * sizeof(T) + (size_t)(D / 32) * 64 * 16; }

template <typename T, int D, bool PAGE16>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void attn_decode_kernel(const DecodeArgs a) {
  typedef Mma<T> M;
  typedef typename M::v8 v8;
  typedef typename M::v4 v4;
  constexpr int LDV = D + 16;  // 32-byte row skew for the transposed reads
  constexpr int NKS = D / 32;
  constexpr int NDT = D / 16;
  constexpr int CH = D / 8;
  constexpr int NLD = 16 * CH / 64;
  extern __shared__ __align__(16) char decode_smem[];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // this wave's LDS: the V tile, then its query fragments
  T* vs = reinterpret_cast<T*>(decode_smem + wv * decode_lds_per_wave<T, D>());
  v8* qs = reinterpret_cast<v8*>(vs + 16 * LDV);
  const int64_t cap = a.tab.cols * a.tab.page;

  const int R = a.Hq / a.Hkv, hgroups = (R + 15) / 16;
  const int kvh = (blockIdx.y / hgroups) * a.kvw + wv;
  const int hcol = (blockIdx.y % hgroups) * 16 + (lane & 15);
  const bool hvalid = hcol < R;
  const int head = kvh * R + (hvalid ? hcol : 0);
  const int grp = lane >> 4;
  const char* kvk = a.k.base + kvh * a.k.sh;
  const char* kvv = a.v.base + kvh * a.v.sh;
  const uint64_t ksb = (uint32_t)a.k.sb, vsb = (uint32_t)a.v.sb;
  const float c = a.c > 0.f ? a.c : (a.c < 0.f ? -a.c : 1.f);

  // keys [k_lo, k_hi) of sequence b (k_lo a multiple of 16); the result goes
  // to the output (slot < 0) or to workspace slot `slot`
  auto piece = [&](int64_t b, int64_t k_lo, int64_t k_hi, int64_t slot) {
    const int ntiles = k_hi > k_lo ? (int)((k_hi - k_lo + 15) / 16) : 0;
    // query fragments (B operand of S^T): lane holds head column lane % 16,
    // dims 32 s + 8 grp .. +7; kept in LDS to leave registers for two tiles
    // in flight (the previous piece's reads of them were issued earlier by
    // this wave, and LDS operations of a wave complete in order)
    {
      const T* qp = reinterpret_cast<const T*>(a.q) + b * a.q_ss + (int64_t)head * a.q_sh + 8 * grp;
      // a negative scale is folded into q (an exact sign flip), a zero scale
      // is q = 0 with c = 1 (equal weights), so the softmax below has c > 0
#pragma unroll
      for (int s = 0; s < NKS; ++s) {
        const v8 qv = hvalid ? *reinterpret_cast<const v8*>(qp + 32 * s) : v8{};
        qs[s * 64 + lane] = a.c > 0.f ? qv : (a.c < 0.f ? -qv : v8{});
      }
    }

    // block id of tile t's page (PAGE16), -1 past the range or for an entry
    // outside [0, num_blocks)
    // (PAGE16: the sequence's table row is found once; a tile is 16-key
    // group g0 + t, in page g / gpp at slot 16 (g % gpp); key positions,
    // table columns and block-offset products fit 32 bits, which the
    // launcher checks, so no 64-bit division or product is left per tile)
    const void* trow = PAGE16 ? reinterpret_cast<const char*>(a.tab.table) +
                                    (a.tab.is64 ? 8 : 4) * (b * a.tab.row_stride)
                              : nullptr;
    const uint32_t gpp = PAGE16 ? (uint32_t)a.tab.page / 16u : 1u;
    const uint32_t g0 = (uint32_t)k_lo / 16u;
    auto tile_block = [&](int t) -> int64_t {
      if (!PAGE16 || t >= ntiles) return -1;
      const uint32_t g = g0 + (uint32_t)t;
      const uint32_t col = gpp == 1u ? g : g / gpp;
      const int64_t blk = load_index_scalar(trow, col, a.tab.is64);
      return blk >= 0 && blk < a.tab.num_blocks ? blk : -1;
    };
    // row r of tile t
    auto row_ptr = [&](const KvSource& src, int t, int64_t blk, int r) -> const char* {
      const int64_t j = k_lo + 16 * (int64_t)t + r;
      if (j >= k_hi) return nullptr;
      if (PAGE16) {
        if (blk < 0) return nullptr;
        return src.base + blk * src.sb + (j % a.tab.page) * src.st + kvh * src.sh;
      }
      return kv_row<true>(src, a.tab, b, 0, j, kvh);
    };
    auto load_tile = [&](int t, int64_t blk, uint4* kd, uint4* vd) {
      if (PAGE16) {
        // one page per tile: buffer loads through a descriptor of this kv
        // head's rows of the page (32-bit offsets, rows past the range read 0)
        const uint32_t j0 = (uint32_t)k_lo + 16u * (uint32_t)t;
        const int32_t nv = t < ntiles ? (int32_t)((uint32_t)k_hi - j0) : 0;
        const uint32_t nvalid = blk < 0 ? 0u : (uint32_t)(nv < 16 ? nv : 16);
        const uint32_t g = g0 + (uint32_t)t;
        const uint32_t r0 = gpp == 1u ? 0u : 16u * (g - (g / gpp) * gpp);
        const uint64_t bb = blk < 0 ? 0u : (uint32_t)blk;
        // the ranges end after the tile's valid rows in the page, so the
        // rows past them read as zero with no test per row
        const uint32_t kst = (uint32_t)a.k.st, vst = (uint32_t)a.v.st;
        const __amdgpu_buffer_rsrc_t rk =
            __builtin_amdgcn_make_buffer_rsrc((void*)(kvk + bb * ksb), 0, (r0 + nvalid) * kst, 0x00020000);
        const __amdgpu_buffer_rsrc_t rv =
            __builtin_amdgcn_make_buffer_rsrc((void*)(kvv + bb * vsb), 0, (r0 + nvalid) * vst, 0x00020000);
        const uint32_t ko = (r0 + (uint32_t)(lane & 15)) * kst + 16u * grp;
#pragma unroll
        for (int s = 0; s < NKS; ++s)
          kd[s] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, ko + 64u * s, 0, 0));
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
          const uint32_t cc = lane + 64 * i, row = cc / CH, ch = cc % CH;
          vd[i] =
              __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, (r0 + row) * vst + 16u * ch, 0, 0));
        }
        return;
      }
      {
        const char* pk = row_ptr(a.k, t, blk, lane & 15);
#pragma unroll
        for (int s = 0; s < NKS; ++s)
          kd[s] = pk ? *reinterpret_cast<const uint4*>(pk + 2 * (32 * s + 8 * grp)) : uint4{0, 0, 0, 0};
      }
#pragma unroll
      for (int i = 0; i < NLD; ++i) {
        const int cc = lane + 64 * i, row = cc / CH, ch = cc % CH;
        const char* pv = row_ptr(a.v, t, blk, row);
        vd[i] = pv ? *reinterpret_cast<const uint4*>(pv + 16 * ch) : uint4{0, 0, 0, 0};
      }
    };

    f32x4 oacc[NDT];
#pragma unroll
    for (int d = 0; d < NDT; ++d) oacc[d] = f32x4{};
    float m_used = -INFINITY, lsum = 0.f;
    float nb = 0.f;  // -m_used, or 0 while m_used is -inf (the exponent offset)

    // first half of a tile: its V rows to LDS (the previous tile's transposed
    // reads were issued earlier by this wave, and LDS operations of a wave
    // complete in order) and its scores; the tile's registers are free after it
    auto scores = [&](const uint4* kd, const uint4* vd) -> f32x4 {
#pragma unroll
      for (int i = 0; i < NLD; ++i) {
        const int cc = lane + 64 * i, row = cc / CH, ch = cc % CH;
        *reinterpret_cast<uint4*>(&vs[row * LDV + 8 * ch]) = vd[i];
      }
      // the query fragments are re-read from LDS on every tile (an opaque
      // index keeps them from being hoisted into registers)
      int qo = lane;
      asm volatile("" : "+v"(qo));
      f32x4 s = f32x4{};
#pragma unroll
      for (int k = 0; k < NKS; ++k) s = M::m16k32(__builtin_bit_cast(v8, kd[k]), qs[k * 64 + qo], s);
      return s;
    };
    // second half: softmax of the scores (lane holds head column lane % 16,
    // keys 4 grp + r of the tile) and O^T += V^T P^T
    auto accumulate = [&](int t, f32x4 s) {
      const uint32_t j0 = (uint32_t)k_lo + 16u * (uint32_t)t;  // (key positions fit 32 bits)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (j0 + 4u * grp + r >= (uint32_t)k_hi) s[r] = -INFINITY;
      // maximum of this lane's 4 keys (c > 0; masked scores are -inf and give
      // p = 0).  A head's 16 keys of the tile lie in the four 16-lane groups,
      // which share one base: it moves only when some lane's keys exceed it
      // by 2^8, and then to the maximum over the four lanes, taken only on
      // that rare path (the same decisions and bases as taking it every tile)
      const float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
      if (__builtin_amdgcn_ballot_w64(mx * c > m_used + 8.f) != 0) {
        float mg = fmaxf(mx, __shfl_xor(mx, 16));
        mg = fmaxf(mg, __shfl_xor(mg, 32));
        const float mn = fmaxf(m_used, mg * c);
        const float alpha = mn == -INFINITY ? 1.f : exp2_fast(m_used - mn);
#pragma unroll
        for (int d = 0; d < NDT; ++d) oacc[d] *= alpha;
        lsum *= alpha;
        m_used = mn;
        nb = mn == -INFINITY ? 0.f : -mn;
      }
      v4 pf;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = exp2_fast(__builtin_fmaf(s[r], c, nb));
        lsum += p;
        pf[r] = (T)p;
      }
      // V^T fragments: lane holds dv 16 d + lane % 16, keys 4 grp + 0..3
      const int j16 = lane & 15;
      const T* vp = vs + (4 * grp + (j16 >> 2)) * LDV + 4 * (j16 & 3);
#pragma unroll
      for (int d = 0; d < NDT; ++d) oacc[d] = M::m16k16(tr4<v4>(vp + 16 * d), pf, oacc[d]);
    };

    // two tiles in flight: buffers A (even tiles) and B (odd tiles); block
    // ids are looked up two tiles before their loads are issued.  Loads are
    // issued unconditionally (a tile past the range reads zeros and its keys
    // are masked), so no branch makes the compiler drain the loads in flight.
    uint4 kA[NKS], kB[NKS];
    uint4 vA[NLD], vB[NLD];
    int64_t bA = tile_block(2), bB = tile_block(3);
    load_tile(0, tile_block(0), kA, vA);
    load_tile(1, tile_block(1), kB, vB);
    for (int t = 0; t < ntiles; t += 2) {
      f32x4 s = scores(kA, vA);
      load_tile(t + 2, bA, kA, vA);
      bA = tile_block(t + 4);
      accumulate(t, s);
      s = scores(kB, vB);
      load_tile(t + 3, bB, kB, vB);
      bB = tile_block(t + 5);
      accumulate(t + 1, s);
    }

    float lt = lsum + __shfl_xor(lsum, 16);
    lt += __shfl_xor(lt, 32);
    if (!hvalid) return;
    if (slot < 0) {
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      T* op = reinterpret_cast<T*>(a.o) + b * a.o_ss + (int64_t)head * a.o_sh + 4 * grp;
#pragma unroll
      for (int d = 0; d < NDT; ++d) {
        v4 ov;
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = (T)(oacc[d][e] * inv);
        *reinterpret_cast<v4*>(op + 16 * d) = ov;
      }
    } else {
      float* pp = a.part + (slot * a.Hq + head) * (int64_t)(D + 4);
#pragma unroll
      for (int d = 0; d < NDT; ++d) *reinterpret_cast<f32x4*>(pp + 16 * d + 4 * grp) = oacc[d];
      if (grp == 0) {
        pp[D] = m_used;
        pp[D + 1] = lt;
      }
    }
  };

  // with one split, unit z is sequence z; else unit u holds the batch's
  // prices [x0, x1) (they fit 31 bits, which the entry point checks)
  constexpr int32_t SP = kDecodeStartPrice;
  int32_t b = blockIdx.z, x0 = 0, x1 = 0, qb = 0;
  if (a.splits > 1) {
    const int64_t U = (int64_t)a.B * a.units;
    const int64_t u = (int64_t)blockIdx.z * a.units + blockIdx.x;
    if (a.prices_inline) {
      // small batch: every wave sums the prices itself (a lane per sequence,
      // 64 at a time), then finds the sequence holding price x0 in a second
      // pass over the exclusive prefix; the first unit's first wave also
      // writes the prefix for the combine
      auto price = [&](int32_t i) -> int32_t {
        if (i >= a.B) return 0;
        const int32_t t = (int32_t)((clamp64(load_index(a.ctx, i, a.ctx64), 0, cap) + 15) / 16);
        return t > 0 ? t + SP : 0;
      };
      int32_t tot = 0;
      for (int32_t c0 = 0; c0 < a.B; c0 += 64) tot += price(c0 + lane);
#pragma unroll
      for (int d = 1; d < 64; d *= 2) tot += __shfl_xor(tot, d);
      tot = __builtin_amdgcn_readfirstlane(tot);
      x0 = (int32_t)(u * tot / U);
      x1 = (int32_t)((u + 1) * tot / U);
      const bool writer = u == 0 && blockIdx.y == 0 && wv == 0;
      if (writer && lane == 0) a.prices[a.B] = tot;
      if (x0 >= x1 && !writer) return;  // an empty unit (a smaller total than U): no piece
      int32_t run = 0;
      for (int32_t c0 = 0; c0 < a.B; c0 += 64) {
        const int32_t p = price(c0 + lane);
        int32_t inc = p;
#pragma unroll
        for (int d = 1; d < 64; d *= 2) {
          const int32_t y = __shfl_up(inc, d);
          if (lane >= d) inc += y;
        }
        const int32_t ex = run + inc - p;  // Q of sequence c0 + lane
        if (writer && c0 + lane < a.B) a.prices[c0 + lane] = ex;
        // the lanes with Q <= x0 are a prefix of the chunk's sequences
        const int32_t cnt = (int32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(c0 + lane < a.B && ex <= x0));
        if (cnt > 0) {
          b = c0 + cnt - 1;
          qb = __builtin_amdgcn_readlane(ex, cnt - 1);
        }
        run += __builtin_amdgcn_readlane(inc, 63);
        if (cnt < 64 && !writer) break;  // (the answer is in this chunk)
      }
      if (x0 >= x1) return;
    } else {
      const int64_t Pt = load_index_scalar(a.prices, a.B, false);
      x0 = (int32_t)(u * Pt / U);
      x1 = (int32_t)((u + 1) * Pt / U);
      if (x0 >= x1) return;  // an empty unit (a smaller total than U): no piece
      // the sequence holding price x0: the last b < B with Q[b] <= x0 (Q[0] =
      // 0), by a 64-ary search over the prefix (one probe per lane per
      // round, Q[lo] <= x0 throughout)
      int32_t lo = 0, hi = a.B;
      while (hi - lo > 64) {
        const int32_t step = (hi - lo + 63) / 64;
        const int32_t idx = lo + lane * step;
        const bool le = idx < hi && a.prices[idx] <= x0;
        lo += ((int32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(le)) - 1) * step;
        hi = lo + step < hi ? lo + step : hi;
      }
      const int32_t idx = lo + lane;
      const bool le = idx < hi && a.prices[idx] <= x0;
      b = __builtin_amdgcn_readfirstlane(lo + (int32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(le)) - 1);
      qb = (int32_t)load_index_scalar(a.prices, b, false);
    }
  }
  for (;;) {
    const int64_t L = clamp64(load_index(a.ctx, b, a.ctx64), 0, cap);
    // keys of the piece: the whole sequence (one split; a zero row when L =
    // 0), or its tiles whose prices lie in the unit's range.  A unit that
    // holds all of a sequence's tiles writes its output row itself (the
    // combine finds that sequence in one unit and skips it), else the piece
    // goes to its workspace slot.
    int32_t qn = 0;
    int64_t k_lo = 0, k_hi = L, slot = -1;
    bool any = true;
    if (a.splits > 1) {
      const int32_t tb = (int32_t)((L + 15) / 16);  // the sequence's tiles
      qn = qb + (tb > 0 ? tb + SP : 0);
      const int32_t r0 = x0 - qb - SP, r1 = x1 - qb - SP;
      const int32_t t0 = r0 < 0 ? 0 : (r0 > tb ? tb : r0), t1 = r1 < 0 ? 0 : (r1 > tb ? tb : r1);
      k_lo = 16 * (int64_t)t0;
      k_hi = 16 * (int64_t)t1 < L ? 16 * (int64_t)t1 : L;
      any = t1 > t0;
      if (t0 > 0 || t1 < tb) slot = (int64_t)b + (int64_t)blockIdx.z * a.units + blockIdx.x;
    }
    if (any) piece(b, k_lo, k_hi, slot);
    if (a.splits == 1 || qn >= x1) break;
    ++b;
    qb = qn;
  }
}

// Merge of the pieces of one (sequence, query head): one wave, D / 64
// output elements per lane.  Sequence b's tiles, at prices [Q_b + start,
// Q_{b+1}), lie in units u0 = unit(Q_b + start) .. u1 = unit(Q_{b+1} - 1),
// unit(x) = ((x + 1) U - 1) / Q_B (the u with u Q_B / U <= x < (u+1) Q_B / U);
// a unit with an empty price range (only when Q_B < U) holds no piece.  Piece
// (b, u) is workspace slot b + u; a sequence inside one unit has no piece
// there, its row was written by that unit.  The pieces are taken 64 at a time, lane i
// reading piece i's maximum and row sum, so their loads are in flight
// together; the running maximum carries over between groups of 64.
template <typename T, int D>
__global__ __launch_bounds__(64) void attn_decode_combine_kernel(const DecodeArgs a) {
  const int64_t bh = blockIdx.x;  // b * Hq + head
  const int64_t b = bh / a.Hq;
  const int head = (int)(bh % a.Hq);
  const int lane = threadIdx.x;
  constexpr int PS = D + 4;
  constexpr int E = D / 64;
  T* op = reinterpret_cast<T*>(a.o) + b * a.o_ss + (int64_t)head * a.o_sh + E * lane;
  const int64_t U = (int64_t)a.B * a.units;
  const int64_t Pt = load_index_scalar(a.prices, a.B, false), qb = load_index_scalar(a.prices, b, false),
                qn = load_index_scalar(a.prices, b + 1, false);
  float acc[E] = {};
  float l = 0.f;
  if (qn > qb) {  // (else no keys: a zero row)
    const int64_t u0 = ((qb + kDecodeStartPrice + 1) * U - 1) / Pt, u1 = (qn * U - 1) / Pt;
    if (u0 == u1) return;  // one unit held the whole sequence and wrote its row
    const bool all_units = Pt >= U;  // every unit has a price range
    const float* base = a.part + ((b + u0) * a.Hq + head) * (int64_t)PS;
    const int64_t rs = (int64_t)a.Hq * PS;  // one slot further
    float mx = -INFINITY;
    for (int64_t c0 = 0; c0 <= u1 - u0; c0 += 64) {
      const int64_t i = c0 + lane, u = u0 + i;
      const bool ok = u <= u1 && (all_units || (u + 1) * Pt / U > u * Pt / U);
      const float mi = ok ? base[i * rs + D] : -INFINITY;
      const float li = ok ? base[i * rs + D + 1] : 0.f;
      float cm = mi;
#pragma unroll
      for (int d = 1; d < 64; d *= 2) cm = fmaxf(cm, __shfl_xor(cm, d));
      const float mn = fmaxf(mx, cm);
      if (mn == -INFINITY) continue;
      const float sc = exp2_fast(mx - mn);  // (0 while mx is -inf)
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] *= sc;
      l *= sc;
      mx = mn;
      const float wi = mi == -INFINITY ? 0.f : exp2_fast(mi - mx);
      float ls = wi * li;
#pragma unroll
      for (int d = 1; d < 64; d *= 2) ls += __shfl_xor(ls, d);
      l += ls;
      const int cnt = u1 - u0 + 1 - c0 < 64 ? (int)(u1 - u0 + 1 - c0) : 64;
      for (int j = 0; j < cnt; ++j) {
        const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wi), j));
        const float* pp = base + (c0 + j) * rs + E * lane;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const float v = pp[e];
          acc[e] += wj == 0.f ? 0.f : wj * v;  // (an empty unit's slot holds stale data)
        }
      }
    }
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) op[e] = (T)(acc[e] * inv);
}

constexpr float kLog2e = 1.4426950408889634f;

KvSource kv_source(const gdn_tensor* t, bool paged) {
  const int64_t es = t->dtype == GDN_DTYPE_F32 ? 4 : 2;
  KvSource s;
  s.base = reinterpret_cast<const char*>(t->data);
  if (paged) {
    s.sb = t->stride[0] * es;
    s.st = t->stride[1] * es;
    s.sh = t->stride[2] * es;
  } else {
    s.sb = 0;
    s.st = t->stride[0] * es;
    s.sh = t->stride[1] * es;
  }
  return s;
}

PagedTable paged_table(const gdn_tensor* tab, const gdn_tensor* kc) {
  PagedTable p;
  p.table = tab->data;
  p.row_stride = tab->stride[0];
  p.cols = tab->shape[1];
  p.num_blocks = kc->shape[0];
  p.page = (int32_t)kc->shape[1];
  p.is64 = tab->dtype == GDN_DTYPE_I64;
  return p;
}

template <typename T, int D, int BN, bool PAGED>
hipError_t launch_prefill_t(const AttnArgs& a, int64_t nseq, int64_t max_len, hipStream_t st) {
  const int qsubs = 4 / a.gh;
  // output rows no sequence covers are zero, as the reference allocates o
  // zero-filled (ops/full_attention.py:467); a kernel of its own, launched
  // first (a call inside the attention kernel changed its register allocation
  // and cost it about a fifth of its speed)
  zero_uncovered_rows_kernel<(int)sizeof(T)><<<dim3(64), dim3(256), 0, st>>>(a.o, a.o_st, a.o_sh, a.Hq, D, a.cu,
                                                                             a.cu64, a.nseq, a.T);
  if (nseq <= 0 || max_len <= 0) return hipGetLastError();
  // query tiles: at most T / tile_len + one partial tile per sequence
  const int64_t tiles = a.T / (32 * qsubs) + nseq;
  const dim3 grid((unsigned)(tiles * (a.Hq / a.gh)));
  if (!PAGED)
    hipLaunchKernelGGL((attn_prefill_kernel<T, D, BN, 0>), grid, dim3(256), 0, st, a);
  else if (a.tab.page % 16 == 0 && a.k.sb < (int64_t(1) << 32) && a.v.sb < (int64_t(1) << 32) && a.tab.cols > 0 &&
           a.tab.cols * a.tab.page < (int64_t(1) << 31) && a.tab.num_blocks < (int64_t(1) << 31)) {
    // whole 16-row groups per page, 32-bit table arithmetic
    if (a.tab.is64)
      hipLaunchKernelGGL((attn_prefill_kernel<T, D, BN, 3>), grid, dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((attn_prefill_kernel<T, D, BN, 2>), grid, dim3(256), 0, st, a);
  } else
    hipLaunchKernelGGL((attn_prefill_kernel<T, D, BN, 1>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

template <bool PAGED>
hipError_t launch_prefill(const AttnArgs& a, int dtype, int D, int64_t nseq, int64_t max_len, hipStream_t st) {
  if (dtype == GDN_DTYPE_BF16) {
    if (D == 64) return launch_prefill_t<bf16_t, 64, 64, PAGED>(a, nseq, max_len, st);
    if (D == 128) return launch_prefill_t<bf16_t, 128, 64, PAGED>(a, nseq, max_len, st);
    return launch_prefill_t<bf16_t, 256, 32, PAGED>(a, nseq, max_len, st);
  }
  if (D == 64) return launch_prefill_t<f16_t, 64, 64, PAGED>(a, nseq, max_len, st);
  if (D == 128) return launch_prefill_t<f16_t, 128, 64, PAGED>(a, nseq, max_len, st);
  return launch_prefill_t<f16_t, 256, 32, PAGED>(a, nseq, max_len, st);
}

int heads_per_group(int R) { return R % 4 == 0 ? 4 : (R % 2 == 0 ? 2 : 1); }

template <typename T, int D>
hipError_t launch_decode_t(const DecodeArgs& a, hipStream_t st) {
  const int hgroups = (a.Hq / a.Hkv + 15) / 16;
  const dim3 grid((unsigned)(a.splits > 1 ? a.units : 1), (unsigned)(a.Hkv / a.kvw * hgroups), (unsigned)a.B);
  const size_t lds = (size_t)a.kvw * decode_lds_per_wave<T, D>();
  if (a.splits > 1 && !a.prices_inline) {
    attn_decode_prices_kernel<<<dim3(1), dim3(1024), 0, st>>>(a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (a.tab.page % 16 == 0 && a.k.sb < (int64_t(1) << 32) && a.v.sb < (int64_t(1) << 32) &&
      a.tab.cols * a.tab.page < (int64_t(1) << 31) && a.tab.num_blocks < (int64_t(1) << 31))
    hipLaunchKernelGGL((attn_decode_kernel<T, D, true>), grid, dim3(64 * a.kvw), lds, st, a);
  else
    hipLaunchKernelGGL((attn_decode_kernel<T, D, false>), grid, dim3(64 * a.kvw), lds, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.splits == 1) return e;
  hipLaunchKernelGGL((attn_decode_combine_kernel<T, D>), dim3((unsigned)((int64_t)a.B * a.Hq)), dim3(64), 0, st, a);
  return hipGetLastError();
}

}  // namespace

hipError_t attn_varlen_prefill_launch(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v,
                                      const gdn_tensor* cu, gdn_tensor* out, int64_t max_seqlen, float scale,
                                      int causal, hipStream_t st) {
  const int64_t nseq = cu->shape[0] - 1;
  if (q->shape[0] == 0) return hipSuccess;
  AttnArgs a{};
  a.q = q->data;
  a.q_st = q->stride[0];
  a.q_sh = q->stride[1];
  a.k = kv_source(k, false);
  a.v = kv_source(v, false);
  a.o = out->data;
  a.o_st = out->stride[0];
  a.o_sh = out->stride[1];
  a.cu = cu->data;
  a.cu64 = cu->dtype == GDN_DTYPE_I64;
  a.T = q->shape[0];
  a.nseq = nseq;
  a.Hq = (int32_t)q->shape[1];
  a.Hkv = (int32_t)k->shape[1];
  a.gh = heads_per_group(a.Hq / a.Hkv);
  a.c = scale * kLog2e;
  a.causal = causal != 0;
  return launch_prefill<false>(a, q->dtype, (int)q->shape[2], nseq, max_seqlen, st);
}

hipError_t attn_paged_prefill_launch(const gdn_tensor* q, const gdn_tensor* kc, const gdn_tensor* vc,
                                     const gdn_tensor* tab, const gdn_tensor* ctx, const gdn_tensor* cu,
                                     gdn_tensor* out, int64_t max_seqlen, float scale, hipStream_t st) {
  const int64_t nseq = cu->shape[0] - 1;
  if (q->shape[0] == 0) return hipSuccess;
  AttnArgs a{};
  a.q = q->data;
  a.q_st = q->stride[0];
  a.q_sh = q->stride[1];
  a.k = kv_source(kc, true);
  a.v = kv_source(vc, true);
  a.o = out->data;
  a.o_st = out->stride[0];
  a.o_sh = out->stride[1];
  a.cu = cu->data;
  a.cu64 = cu->dtype == GDN_DTYPE_I64;
  a.ctx = ctx->data;
  a.ctx64 = ctx->dtype == GDN_DTYPE_I64;
  a.tab = paged_table(tab, kc);
  a.T = q->shape[0];
  a.nseq = nseq;
  a.Hq = (int32_t)q->shape[1];
  a.Hkv = (int32_t)kc->shape[2];
  a.gh = heads_per_group(a.Hq / a.Hkv);
  a.c = scale * kLog2e;
  a.causal = true;
  return launch_prefill<true>(a, q->dtype, (int)q->shape[2], nseq, max_seqlen, st);
}

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxScratchDevices] = {};
}  // namespace

// Device address of `scratch` on the device that runs stream st, looked up on
// that device's first call (with the device made current for the lookup and
// the caller's current device restored) and cached.
hipError_t attn_decode_scratch(hipStream_t st, float** ptr) {
  int dev = 0;
  hipError_t e = st ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = 0;
    if ((e = hipGetDevice(&cur)) != hipSuccess) return e;
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t r = cur != dev ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess) return e;
    if (r != hipSuccess) return r;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *ptr = g_scratch_ptr[dev];
  return hipSuccess;
}

int32_t attn_decode_start_price() { return kDecodeStartPrice; }

hipError_t attn_paged_decode_launch(const gdn_tensor* q, const gdn_tensor* kc, const gdn_tensor* vc,
                                    const gdn_tensor* tab, const gdn_tensor* ctx, gdn_tensor* out, float* workspace,
                                    int32_t splits, float scale, hipStream_t st) {
  if (q->shape[0] == 0) return hipSuccess;
  DecodeArgs a{};
  a.q = q->data;
  a.q_ss = q->stride[0];
  a.q_sh = q->stride[1];
  a.k = kv_source(kc, true);
  a.v = kv_source(vc, true);
  a.o = out->data;
  a.o_ss = out->stride[0];
  a.o_sh = out->stride[1];
  a.ctx = ctx->data;
  a.ctx64 = ctx->dtype == GDN_DTYPE_I64;
  a.tab = paged_table(tab, kc);
  a.B = (int32_t)q->shape[0];
  a.Hq = (int32_t)q->shape[1];
  a.Hkv = (int32_t)kc->shape[2];
  a.splits = splits;
  a.kvw = a.Hkv % 4 == 0 ? 4 : (a.Hkv % 2 == 0 ? 2 : 1);
  a.c = scale * kLog2e;
  if (splits > 1) {
    // workspace: the pieces' partials, B + U = B splits slots x Hq rows,
    // then the price prefix
    a.units = splits - 1;
    a.part = workspace;
    a.prices = reinterpret_cast<int32_t*>(workspace + (int64_t)a.B * splits * a.Hq * (q->shape[2] + 4));
    // up to 1,024 sequences every decode wave sums the prices itself (16
    // loads per lane) instead of waiting for a launch that writes them
    a.prices_inline = a.B <= 1024;
  }
  const int D = (int)q->shape[2];
  if (q->dtype == GDN_DTYPE_BF16) {
    if (D == 64) return launch_decode_t<bf16_t, 64>(a, st);
    if (D == 128) return launch_decode_t<bf16_t, 128>(a, st);
    return launch_decode_t<bf16_t, 256>(a, st);
  }
  if (D == 64) return launch_decode_t<f16_t, 64>(a, st);
  if (D == 128) return launch_decode_t<f16_t, 128>(a, st);
  return launch_decode_t<f16_t, 256>(a, st);
}
