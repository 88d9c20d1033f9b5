// Building blocks shared by the gfx950 MFMA decode kernels (decode_mfma.hip:
// one workgroup per context partition; decode_sk.hip: persistent workgroups
// over equal shares of all sequences' chunks).
//
// A wavefront processes the context in 32-token chunks. Per chunk it
//   1. stores the chunk's K and V rows, prefetched into registers by 16-byte
//      coalesced loads through the block table, into its private LDS slice
//      (rows padded so the fragment reads below are bank-conflict free);
//   2. issues the loads of the chunk it will process PF chunks later;
//   3. computes S^T = K Q^T with v_mfma_f32_16x16x32 (A = 16 tokens x 32 dims
//      from LDS, B = Q^T in registers), so each K row is read once for all
//      heads of the group;
//   4. updates the online softmax per head in base 2 (each lane owns one head
//      and 8 of the 32 tokens; the row max is a 4-lane xor shuffle);
//   5. computes O^T += V^T P^T with the same instruction: the S^T accumulator
//      layout already is the P^T operand layout (lane = head, 8 tokens), and
//      V^T fragments are gathered from LDS with 16-bit reads.
//
// MFMA operand layouts relied upon (16x16x32, wave64): lane l supplies row
// l%16 of A and column l%16 of B, each with the 8 k-values of group l/16 (the
// k order inside a group is the same for A and B, which is all a reduction
// needs); lane l receives D[4*(l/16) + r][l%16] for r = 0..3.
#pragma once

#include "pkv_internal.h"

namespace pkv {
namespace mfma {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));

// 4 floats times s rounded to T and packed into 8 bytes, and back. Staging
// and split-K partials use the kernel's element type: bf16 keeps fp32's
// exponent range, fp16 holds any weighted mean of fp16 value rows.
template <typename T>
__device__ __forceinline__ uint64_t pack4(floatx4 x, float s) {
  T h[4] = {(T)(x[0] * s), (T)(x[1] * s), (T)(x[2] * s), (T)(x[3] * s)};
  uint64_t b;
  __builtin_memcpy(&b, h, 8);
  return b;
}
template <typename T>
__device__ __forceinline__ floatx4 unpack4(uint64_t b) {
  T h[4];
  __builtin_memcpy(h, &b, 8);
  return floatx4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
}

template <typename T>
struct Ops;
template <>
struct Ops<bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ floatx4 mma(v8 a, v8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Ops<f16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ floatx4 mma(v8 a, v8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
// fp32 operands (the few-row projections of fp32 models): the same lane
// layout as the 16-bit forms (lane l: row l % 16 of A and column l % 16 of
// B, 8 k-values of group l / 16), taken as eight v_mfma_f32_16x16x4_f32
// steps, step j using element j of every lane (k-values j, 8 + j, 16 + j,
// 24 + j of the 32), so each product is an fp32 sum over the same 32 k.
template <>
struct Ops<float> {
  typedef float v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ floatx4 mma(v8 a, v8 b, floatx4 c) {
#pragma unroll
    for (int j = 0; j < 8; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b[j], c, 0, 0, 0);
    return c;
  }
};

// fp8 pools: widening to bf16 / fp16 is exact; gfx950's
// v_cvt_scalef32_pk_{bf16,f16}_fp8 with scale 1 turns two fp8 bytes into two
// 16-bit values. Narrowing (new rows) is f32_to_e4m3.
template <typename T>
struct Fp8;
template <>
struct Fp8<bf16> {
  // bytes 0-1 / 2-3 of w as two bf16 (low half = the lower byte)
  static __device__ __forceinline__ unsigned lo2(unsigned w) {
    return __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
  }
  static __device__ __forceinline__ unsigned hi2(unsigned w) {
    return __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
  }
  static __device__ __forceinline__ float to_f32(unsigned short h) {
    return __uint_as_float((unsigned)h << 16);
  }
};
template <>
struct Fp8<f16> {
  static __device__ __forceinline__ unsigned lo2(unsigned w) {
    return __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
  }
  static __device__ __forceinline__ unsigned hi2(unsigned w) {
    return __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true));
  }
  static __device__ __forceinline__ float to_f32(unsigned short h) {
    return (float)__builtin_bit_cast(_Float16, h);
  }
};

// 8 fp8 values (8 bytes) -> 8 values of T (16 bytes), element order kept
template <typename T>
__device__ __forceinline__ u32x4 widen8(u32x2 p) {
  return u32x4{Fp8<T>::lo2(p.x), Fp8<T>::hi2(p.x), Fp8<T>::lo2(p.y), Fp8<T>::hi2(p.y)};
}
// 8 values of T -> 8 fp8 values, rounded as f32_to_e4m3
template <typename T>
__device__ __forceinline__ u32x2 narrow8(u32x4 p) {
  unsigned out[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const unsigned short h = (unsigned short)(p[e >> 1] >> (16 * (e & 1)));
    out[e >> 2] |= f32_to_e4m3(Fp8<T>::to_f32(h)) << (8 * (e & 3));
  }
  return u32x2{out[0], out[1]};
}

// One 16-byte piece (8 elements) of a K or V row as loaded from the pool:
// 16 bytes from a 16-bit pool, 8 from an fp8 pool.
template <bool KV8>
struct PoolPiece {
  typedef u32x4 type;
  static constexpr int kBytes = 16;
};
template <>
struct PoolPiece<true> {
  typedef u32x2 type;
  static constexpr int kBytes = 8;
};

constexpr int kTblCap = 256;  // block-table entries staged in LDS at a time
constexpr float kLazy = 8.f;  // log2 headroom of the lazily moved softmax reference
constexpr float kLn2f = 0.6931471805599453f;

// 2^x by the hardware's v_exp_f32 alone (the library exp2f adds a rescaling
// for results below 2^-126). Softmax weights that small are below bf16/fp16
// resolution next to the weight-1 term every row holds; -inf gives 0.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// LDS geometry of one 32-token chunk of K (or V) rows, D bf16/fp16 each.
// Rows are padded by 16 bytes (PITCH = 2D + 16): row r starts 4r (mod 64)
// banks further on for D = 128 (36r for D = 64), so the 16 rows an MFMA
// fragment read touches at one 16-byte piece land on distinct bank groups,
// and so do the 4 row groups of a V^T gather. Every fragment address is then
// one base register plus an immediate offset.
template <int D>
struct ChunkGeo {
  static constexpr int CPR = D / 8;                 // 16-byte pieces per row
  static constexpr int ROW_BYTES = D * 2;
  static constexpr int PITCH = ROW_BYTES + 16;
  static constexpr int ROWS_PER_LOAD = 64 / CPR;    // rows one wave load covers
  static constexpr int NPL = kChunk / ROWS_PER_LOAD;  // loads per lane per tensor
  static constexpr int BYTES = kChunk * PITCH;
  static_assert(ROWS_PER_LOAD >= 1 && 64 % CPR == 0, "D must be 64 or 128");
  static __device__ __forceinline__ int off(int r, int c) { return r * PITCH + (c << 4); }
};

// K and V rows of one 32-token chunk held in registers between their loads
// and their LDS stores (as loaded: fp8 bytes from an fp8 pool); bit j of
// `valid` clears row load j (bad table entry).
template <int NPL, bool KV8>
struct ChunkRegs {
  typename PoolPiece<KV8>::type k[NPL];
  typename PoolPiece<KV8>::type v[NPL];
  unsigned valid;
};

// Pool addressing shared by all chunks of a wavefront.
struct PoolView {
  const char* kbase;
  const char* vbase;
  int64_t row_stride;  // bytes per pool slot (hkv * d * element bytes)
  int64_t head_off;    // byte offset of this kv head inside a slot
  int num_blocks;
  int bs_shift;
};

// Where a wavefront is in the current run of chunks: its LDS slices, the
// block-table window staged in LDS, and the token range [seg_lo, seg_hi).
struct ChunkCtx {
  char* kl;
  char* vl;
  const int* tbl;
  int blk_lo;
  int seg_lo;
  int seg_hi;
  int prow;  // first row this lane loads
  int pcol;  // its 16-byte piece within the row
  int grp;   // MFMA k-group of this lane (lane / 16)
  int l16;   // lane % 16
  float scale_log2;
};

// Branch-free loads of chunk `c` (tokens seg_lo + 32c ...): rows past
// seg_hi re-read rows inside the range (their scores are masked to -inf, so
// they contribute exactly 0); rows whose table entry is outside the pool
// read block 0 and are zeroed when staged. Nothing here consumes a load
// result, so the loads stay in flight until the chunk is staged.
//
// HALVES (block size >= 16, chunk starts 16-aligned): each 16-row half of
// the chunk lies in one block, so a half costs one table read and is read
// through a buffer resource of its own (uniform: base = the half's first
// row, size = 16 rows, or 0 for a bad table entry, which makes every load of
// the half return zeros without touching memory); each lane adds only its
// row and piece offset (one min and one multiply-add per load). A half that
// lies wholly past seg_hi re-reads the first half. Otherwise every row
// reads its own table entry and forms a 64-bit address, and bad rows are
// zeroed when staged.
template <bool KV8>
__device__ __forceinline__ typename PoolPiece<KV8>::type load_piece(__amdgpu_buffer_rsrc_t rs,
                                                                    unsigned off) {
  constexpr int kNonTemporal = 2;
  if constexpr (KV8)
    return __builtin_bit_cast(u32x2,
                              __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, kNonTemporal));
  else
    return __builtin_bit_cast(u32x4,
                              __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kNonTemporal));
}
constexpr int kRsrcWord3 = 0x00020000;  // raw (untyped) dword buffer, gfx9 family

template <class Geo, int NPL, bool HALVES, bool KV8>
__device__ __forceinline__ void load_chunk(ChunkRegs<NPL, KV8>& r, const PoolView& pv,
                                           const ChunkCtx& cx, int c) {
  typedef typename PoolPiece<KV8>::type P;
  constexpr int PB = PoolPiece<KV8>::kBytes;
  const int bs_mask = (1 << pv.bs_shift) - 1;
  const int cb = cx.seg_lo + c * kChunk;
  unsigned vmask = 0;
  if constexpr (HALVES) {
    constexpr int LPH = NPL / 2;  // loads per 16-row half
    static_assert(LPH * Geo::ROWS_PER_LOAD == 16, "a half is 16 rows");
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int hs = cb + 16 * h < cx.seg_hi ? cb + 16 * h : cb;
      const int lim = max(0, min(15, cx.seg_hi - 1 - hs));  // last row of the half in range
      const int phys = __builtin_amdgcn_readfirstlane(cx.tbl[(hs >> pv.bs_shift) - cx.blk_lo]);
      const bool ok = (unsigned)phys < (unsigned)pv.num_blocks;
      const int64_t base =
          ((((int64_t)(ok ? phys : 0)) << pv.bs_shift) + (hs & bs_mask)) * pv.row_stride +
          pv.head_off;
      const int extent = ok ? 16 * (int)pv.row_stride : 0;
      const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<char*>(pv.kbase + base), (short)0, extent, kRsrcWord3);
      const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<char*>(pv.vbase + base), (short)0, extent, kRsrcWord3);
#pragma unroll
      for (int j = 0; j < LPH; ++j) {
        const int row = min(cx.prow + j * Geo::ROWS_PER_LOAD, lim);
        const unsigned off = (unsigned)row * (unsigned)pv.row_stride + (unsigned)(cx.pcol * PB);
        r.k[h * LPH + j] = load_piece<KV8>(kr, off);
        r.v[h * LPH + j] = load_piece<KV8>(vr, off);
      }
      vmask |= (ok ? (1u << LPH) - 1 : 0u) << (h * LPH);
    }
  } else {
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      int pos = cb + cx.prow + j * Geo::ROWS_PER_LOAD;
      pos = pos < cx.seg_hi ? pos : cx.seg_hi - 1;
      pos = pos > 0 ? pos : 0;  // an empty context (seg_hi = 0) reads row 0
      const int phys = cx.tbl[(pos >> pv.bs_shift) - cx.blk_lo];
      const bool ok = (unsigned)phys < (unsigned)pv.num_blocks;
      vmask |= (unsigned)ok << j;
      const int64_t slot = ((int64_t)(ok ? phys : 0) << pv.bs_shift) + (pos & bs_mask);
      const int64_t off = slot * pv.row_stride + pv.head_off + cx.pcol * PB;
      r.k[j] = __builtin_nontemporal_load(reinterpret_cast<const P*>(pv.kbase + off));
      r.v[j] = __builtin_nontemporal_load(reinterpret_cast<const P*>(pv.vbase + off));
    }
  }
  r.valid = vmask;
}

// Max / sum over the four lanes of a head (lanes l, l + 16, l + 32, l + 48)
// by the cross-row swaps of gfx950 (v_permlane16_swap, v_permlane32_swap:
// VALU data movement, no LDS round trip). After a swap of x with itself the
// two results hold rows (0, 0, 2, 2) and (1, 1, 3, 3) (resp. halves
// (lo, lo) and (hi, hi)), so every lane combines the same operands in the
// same order and all four end with identical bits.
__device__ __forceinline__ float head_lanes_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float head_lanes_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Online-softmax state of one wavefront: lane l holds head 16*nt + l%16,
// output dims 16*dt + 4*(l/16) + 0..3.
template <int NT, int DT>
struct WaveState {
  floatx4 o[NT][DT];
  float m[NT];
  float l[NT];
  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      m[nt] = -INFINITY;
      l[nt] = 0.f;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[nt][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
  }
};

// The row appended this step (fused append): token position `pos` (-1: none
// in this range), its K and V rows staged in LDS at lds (K: ROW_BYTES bytes,
// then V).
struct NewRow {
  int pos;
  const char* lds;
};

// Overwrites the staged row of token nr.pos when it lies in the chunk that
// starts at token cb (its pool row may not be written yet). With an fp8 pool
// the row is rounded to fp8 and widened back: attention sees the values the
// pool will hold.
template <typename T, class Geo, bool KV8>
__device__ __forceinline__ void stage_new_row(const NewRow& nr, int cb, const ChunkCtx& cx,
                                              int lane) {
  if (nr.pos >= cb && nr.pos < cb + kChunk) {  // uniform across the wavefront
    const int r = nr.pos - cb;
    if (lane < 2 * Geo::CPR) {
      u32x4 x = *reinterpret_cast<const u32x4*>(nr.lds + lane * 16);
      if constexpr (KV8) x = widen8<T>(narrow8<T>(x));
      char* dst = lane < Geo::CPR ? cx.kl + Geo::off(r, lane)
                                  : cx.vl + Geo::off(r, lane - Geo::CPR);
      *reinterpret_cast<u32x4*>(dst) = x;
    }
  }
}

// Registers -> this wavefront's LDS slice, widened to T from an fp8 pool
// (rows with a bad table entry are zeroed and flagged).
// ZEROED: the loads already returned zeros for bad rows (HALVES loads).
template <typename T, class Geo, int NPL, bool KV8, bool ZEROED>
__device__ __forceinline__ void stage_chunk(const ChunkRegs<NPL, KV8>& r, const ChunkCtx& cx,
                                            bool& bad_block) {
  asm volatile("" ::: "memory");
  constexpr unsigned kAll = (1u << NPL) - 1;
  if constexpr (ZEROED) bad_block |= r.valid != kAll;
  // every row valid (the rule) on every lane: plain stores, no selects
  const bool all_ok = ZEROED || __builtin_amdgcn_ballot_w64(r.valid != kAll) == 0;
  const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int row = cx.prow + j * Geo::ROWS_PER_LOAD;
    u32x4 kp, vp;
    if constexpr (KV8) {
      kp = widen8<T>(r.k[j]);
      vp = widen8<T>(r.v[j]);
    } else {
      kp = r.k[j];
      vp = r.v[j];
    }
    if (!all_ok) {
      const bool ok = (r.valid >> j) & 1;
      bad_block |= !ok;
      kp = ok ? kp : zero;
      vp = ok ? vp : zero;
    }
    *reinterpret_cast<u32x4*>(cx.kl + Geo::off(row, cx.pcol)) = kp;
    *reinterpret_cast<u32x4*>(cx.vl + Geo::off(row, cx.pcol)) = vp;
  }
}

// S^T = K Q^T of the chunk staged in cx's K slice: tokens 16h + 4*grp + r
// of the chunk for head 16nt + l16, for the NC row tiles N0 ... of qf (each
// K fragment is read once for all of them).
template <typename T, int D, int NT, int N0, int NC>
__device__ __forceinline__ void chunk_scores_sub(const ChunkCtx& cx,
                                                 const typename Ops<T>::v8 (&qf)[NT][D / 32],
                                                 floatx4 (&sacc)[NC][2]) {
  using Geo = ChunkGeo<D>;
  using v8 = typename Ops<T>::v8;
  constexpr int KS = D / 32;
  static_assert(N0 >= 0 && NC >= 1 && N0 + NC <= NT, "row tiles");
  // the slice is private to this wavefront: waiting for its own LDS writes
  // is the only synchronisation the reads below need
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  // k-step outermost: one K fragment live at a time (each accumulator still
  // sums its k-steps in order 0, 1, ...)
#pragma unroll
  for (int nt = 0; nt < NC; ++nt)
#pragma unroll
    for (int h = 0; h < 2; ++h) sacc[nt][h] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const v8 kf =
          *reinterpret_cast<const v8*>(cx.kl + Geo::off(16 * h + cx.l16, 4 * ks + cx.grp));
#pragma unroll
      for (int nt = 0; nt < NC; ++nt)
        sacc[nt][h] = Ops<T>::mma(kf, qf[N0 + nt][ks], sacc[nt][h]);
    }
  }
}
template <typename T, int D, int NT>
__device__ __forceinline__ void chunk_scores(const ChunkCtx& cx,
                                             const typename Ops<T>::v8 (&qf)[NT][D / 32],
                                             floatx4 (&sacc)[NT][2]) {
  chunk_scores_sub<T, D, NT, 0, NT>(cx, qf, sacc);
}

// Softmax update and O^T += V^T P^T for the chunk whose scores are sacc
// (row tiles N0 ... N0 + NC - 1 of st): tokens seg_lo + 32c ..., those at or
// past seg_hi[nt] masked out for row tile N0 + nt (each V^T fragment is
// read once for all of them).
template <typename T, int D, int NT, int N0, int NC, bool MASK>
__device__ __forceinline__ void chunk_update_sub(int c, const ChunkCtx& cx,
                                                 const int (&seg_hi)[NC],
                                                 const floatx4 (&sacc)[NC][2],
                                                 WaveState<NT, D / 16>& st) {
  using Geo = ChunkGeo<D>;
  using v8 = typename Ops<T>::v8;
  constexpr int DT = D / 16;

  // online softmax (base 2) with a lazily moved reference: probabilities
  // are taken relative to st.m, which only moves (with the head-wide max
  // shuffles and the rescale of l and O) when some score of the wavefront
  // exceeds it by more than kLazy; so p <= 2^kLazy, exact in bf16/fp16
  // relative terms, and most chunks skip the shuffles and the rescale.
  // P^T operand = this lane's 8 probabilities. The scores stay unscaled
  // (masked ones -inf): the scale c = softmax scale * log2(e) > 0 is applied
  // to the row maximum (max(s) c = max(s c) exactly, rounding being
  // monotone) and inside each exponent's fma, p = 2^(s c - m).
  const int cb = cx.seg_lo + c * kChunk;
  const float sc = cx.scale_log2;
  float sv[NC][8];
  bool move = false;
#pragma unroll
  for (int nt = 0; nt < NC; ++nt) {
    // token 16h + 4 grp + rr of the chunk is in range iff 16h + rr < lim
    const int lim = seg_hi[nt] - cb - 4 * cx.grp;
    float mx = -INFINITY;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const float x = !MASK || 16 * h + rr < lim ? sacc[nt][h][rr] : -INFINITY;
        sv[nt][4 * h + rr] = x;
        mx = fmaxf(mx, x);
      }
    move |= mx * sc > st.m[N0 + nt] + kLazy;  // also true on the first scores (m = -inf)
  }
  if (__builtin_amdgcn_ballot_w64(move) != 0) {
#pragma unroll
    for (int nt = 0; nt < NC; ++nt) {
      float mx = -INFINITY;
#pragma unroll
      for (int e = 0; e < 8; ++e) mx = fmaxf(mx, sv[nt][e]);
      mx = head_lanes_max(mx) * sc;
      const float m_new = fmaxf(st.m[N0 + nt], mx);
      const float alpha = m_new == -INFINITY ? 1.f : exp2_fast(st.m[N0 + nt] - m_new);
      st.l[N0 + nt] *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) st.o[N0 + nt][dt] *= alpha;
      st.m[N0 + nt] = m_new;
    }
  }
  v8 pf[NC];
#pragma unroll
  for (int nt = 0; nt < NC; ++nt) {
    const float nref = st.m[N0 + nt] == -INFINITY ? 0.f : -st.m[N0 + nt];
    float ps = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = exp2_fast(__builtin_fmaf(sv[nt][e], sc, nref));
      ps += p;
      pf[nt][e] = (T)p;
    }
    st.l[N0 + nt] += ps;
  }

  // O^T += V^T P^T; V^T fragment: dims 16dt + l16, the same 8 tokens
  // (4grp + e and 16 + 4grp + e), read out of the row-major chunk by two
  // gfx950 transposing LDS reads. ds_read_b64_tr_b16 treats the four
  // 16-bit values each lane of a 16-lane group addresses as a 16 x 4 matrix
  // and returns lane 4i + c the values c of source lanes i, 4 + i, 8 + i,
  // 12 + i; so source lane s addresses token row 4grp + s / 4 (and 16 rows
  // further for the second read), dims 16dt + 4 (s % 4) ... + 3.
  const char* vt = cx.vl + (4 * cx.grp + (cx.l16 >> 2)) * Geo::PITCH + 8 * (cx.l16 & 3);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4s*)(vt + 32 * dt));
    const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4s*)(vt + 32 * dt + 16 * Geo::PITCH));
    const v8s both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    v8 vf;
    __builtin_memcpy(&vf, &both, 16);
#pragma unroll
    for (int nt = 0; nt < NC; ++nt)
      st.o[N0 + nt][dt] = Ops<T>::mma(vf, pf[nt], st.o[N0 + nt][dt]);
  }
}
template <typename T, int D, int NT, bool MASK>
__device__ __forceinline__ void chunk_update(int c, const ChunkCtx& cx,
                                             const floatx4 (&sacc)[NT][2],
                                             WaveState<NT, D / 16>& st) {
  int seg_hi[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) seg_hi[nt] = cx.seg_hi;
  chunk_update_sub<T, D, NT, 0, NT, MASK>(c, cx, seg_hi, sacc, st);
}

// QK / softmax / PV of the chunk staged in cx's slices.
// MASK = false: the chunk lies wholly inside [seg_lo, seg_hi).
template <typename T, int D, int NT, bool MASK = true>
__device__ __forceinline__ void compute_chunk(int c, const ChunkCtx& cx,
                                              const typename Ops<T>::v8 (&qf)[NT][D / 32],
                                              WaveState<NT, D / 16>& st) {
  floatx4 sacc[NT][2];
  chunk_scores<T, D, NT>(cx, qf, sacc);
  chunk_update<T, D, NT, MASK>(c, cx, sacc, st);
}

// One chunk: registers -> LDS slice, optionally refill the registers with
// chunk `c + ahead` (issued before any compute so the loads overlap it),
// then QK / softmax / PV out of LDS.
template <typename T, int D, int NT, int NPL, bool HALVES, bool APP, bool KV8, bool MASK>
__device__ __forceinline__ void chunk_step(
    ChunkRegs<NPL, KV8>& r, int c, bool refill, int ahead, const ChunkCtx& cx,
    const PoolView& pv, const typename Ops<T>::v8 (&qf)[NT][D / 32],
    WaveState<NT, D / 16>& st, bool& bad_block, const NewRow& nr) {
  using Geo = ChunkGeo<D>;
  stage_chunk<T, Geo, NPL, KV8, HALVES>(r, cx, bad_block);
  if constexpr (APP)
    stage_new_row<T, Geo, KV8>(nr, cx.seg_lo + c * kChunk, cx, (int)(threadIdx.x & 63));
  if (refill) load_chunk<Geo, NPL, HALVES, KV8>(r, pv, cx, c + ahead);
  compute_chunk<T, D, NT, MASK>(c, cx, qf, st);
}

// All chunks of [cx.seg_lo, cx.seg_hi) assigned to wavefront w of nw:
// chunks w, w + nw, ... with PF chunks in flight per wavefront (APP: the
// appended row nr is staged over its pool row where it falls). A
// steady-state loop with no data-dependent branch keeps the compiler's wait
// counts exact (staging buffer b waits only for buffer b's loads). Only the
// last chunk of the range can be partial, and the steady-state loop never
// reaches it (its chunks are below nchunks - nw PF), so it skips the mask.
template <typename T, int D, int NT, int PF, bool HALVES, bool APP, bool KV8>
__device__ __forceinline__ void run_chunks(int w, int nw, const ChunkCtx& cx,
                                           const PoolView& pv,
                                           const typename Ops<T>::v8 (&qf)[NT][D / 32],
                                           WaveState<NT, D / 16>& st, bool& bad_block,
                                           const NewRow& nr) {
  using Geo = ChunkGeo<D>;
  constexpr int NPL = Geo::NPL;
  const int nchunks = (cx.seg_hi - cx.seg_lo + kChunk - 1) / kChunk;
  const int step = nw * PF;
  ChunkRegs<NPL, KV8> rb[PF];
#pragma unroll
  for (int b = 0; b < PF; ++b)
    if (w + nw * b < nchunks) load_chunk<Geo, NPL, HALVES, KV8>(rb[b], pv, cx, w + nw * b);
  int c = w;
  for (; c + nw * (2 * PF - 1) < nchunks; c += step) {
#pragma unroll
    for (int b = 0; b < PF; ++b)
      chunk_step<T, D, NT, NPL, HALVES, APP, KV8, false>(rb[b], c + nw * b, true, step, cx, pv,
                                                         qf, st, bad_block, nr);
  }
#pragma unroll
  for (int b = 0; b < PF; ++b)
    if (c + nw * b < nchunks)
      chunk_step<T, D, NT, NPL, HALVES, APP, KV8, true>(
          rb[b], c + nw * b, c + nw * (b + PF) < nchunks, step, cx, pv, qf, st, bad_block, nr);
  c += step;
#pragma unroll
  for (int b = 0; b < PF; ++b)
    if (c + nw * b < nchunks)
      chunk_step<T, D, NT, NPL, HALVES, APP, KV8, true>(rb[b], c + nw * b, false, step, cx, pv,
                                                        qf, st, bad_block, nr);
}

// Combination of the NW wavefronts' online-softmax states of one
// (sequence, kv head) after they are staged in LDS: ob = [NW][G][D + 4]
// floats (O of each wavefront), ml = [NW][G] (m, l). Thread tid of BLOCK
// owns head tid / TPH and the float4 columns cq + TPH q (q < NQ), so the
// softmax weights of the wavefronts, the sum and its reciprocal are taken
// once per head and thread rather than once per output column, and
// consecutive threads read and write consecutive columns.
template <int G, int D, int NW, int BLOCK>
struct WaveCombine {
  static constexpr int TPH = BLOCK / G;        // threads per head
  static constexpr int NQ = D / (4 * TPH);     // float4 columns per thread
  static constexpr int OPITCH = D + 4;
  static_assert(BLOCK % G == 0 && NQ >= 1 && D % (4 * TPH) == 0, "block / head split");
  int head, cq;
  float M, L, inv;  // running max (base 2), sum, 1 / sum (0 when the sum is 0)
  floatx4 acc[NQ];  // unnormalised output columns

  __device__ __forceinline__ int col(int q) const { return 4 * (cq + TPH * q); }

  __device__ __forceinline__ void run(const float* ob, const float (*ml)[G][2], int tid) {
    head = tid / TPH;
    cq = tid - head * TPH;
    M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, ml[ww][head][0]);
    L = 0.f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) acc[q] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (M != -INFINITY) {
      float wt[NW];
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) {
        wt[ww] = exp2f(ml[ww][head][0] - M);
        L += ml[ww][head][1] * wt[ww];
      }
#pragma unroll
      for (int ww = 0; ww < NW; ++ww)
#pragma unroll
        for (int q = 0; q < NQ; ++q)
          acc[q] += wt[ww] * *reinterpret_cast<const floatx4*>(ob + (ww * G + head) * OPITCH + col(q));
    }
    inv = L > 0.f ? 1.f / L : 0.f;
  }
};

// The same combination with the wavefront states staged as O / l rounded to
// the 16-bit element type S (half the LDS bytes of fp32 O; each is a
// weighted mean of value rows, so within their range): ob = [NW][G][OPITCH]
// values of S, ml = [NW][G] (m, l). Wavefront ww's weight is
// l_ww 2^(m_ww - M).
template <typename S, int G, int D, int NW, int BLOCK>
struct WaveCombine16 {
  static constexpr int TPH = BLOCK / G;        // threads per head
  static constexpr int NQ = D / (4 * TPH);     // 4-column groups per thread
  static constexpr int OPITCH = D + 8;         // values of S
  static_assert(BLOCK % G == 0 && NQ >= 1 && D % (4 * TPH) == 0, "block / head split");
  int head, cq;
  float M, L, inv;  // running max (base 2), sum, 1 / sum (0 when the sum is 0)
  floatx4 acc[NQ];  // unnormalised output columns

  __device__ __forceinline__ int col(int q) const { return 4 * (cq + TPH * q); }

  __device__ __forceinline__ void run(const S* ob, const float (*ml)[G][2], int tid) {
    head = tid / TPH;
    cq = tid - head * TPH;
    M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, ml[ww][head][0]);
    L = 0.f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) acc[q] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (M != -INFINITY) {
      float wt[NW];
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) {
        wt[ww] = ml[ww][head][1] * exp2f(ml[ww][head][0] - M);
        L += wt[ww];
      }
#pragma unroll
      for (int ww = 0; ww < NW; ++ww)
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          acc[q] += wt[ww] * unpack4<S>(
                                 *reinterpret_cast<const uint64_t*>(ob + (ww * G + head) * OPITCH + col(q)));
        }
    }
    inv = L > 0.f ? 1.f / L : 0.f;
  }
};

// Fused append of one sequence's query-token row. load_new_row /
// put_new_row: threads [0, 2 CPR) of the workgroup copy their 16-byte piece
// of the K / V row `tok` (kv head `kvh`) into the LDS row buffer (the
// caller's barrier publishes it). store_new_row: the same threads write it
// into the pool slot of
// position pos, after the table and pool checks of the stand-alone append
// (whose status bits are raised instead of writing); the table entry comes
// from the LDS table window tbl (blocks blk_lo ...) when it covers pos.
// Every thread loads a piece (threads past 2 CPR a duplicate, so no load
// sits under a branch); put_new_row then stores threads [0, 2 CPR)'s pieces.
template <int D>
__device__ __forceinline__ u32x4 load_new_row(const AttnArgs& a, int tok, int kvh, int tid) {
  using Geo = ChunkGeo<D>;
  const int t = tid % (2 * Geo::CPR);
  const bool is_v = t >= Geo::CPR;
  const int64_t off = ((int64_t)tok * a.hkv + kvh) * D * 2 + (t % Geo::CPR) * 16;
  return *reinterpret_cast<const u32x4*>(static_cast<const char*>(is_v ? a.v_new : a.k_new) +
                                         off);
}

template <int D>
__device__ __forceinline__ void put_new_row(char* lds, u32x4 piece, int tid) {
  if (tid < 2 * ChunkGeo<D>::CPR) *reinterpret_cast<u32x4*>(lds + tid * 16) = piece;
}

template <typename T, int D, bool KV8>
__device__ __forceinline__ void store_new_row(const char* lds, const AttnArgs& a, int s,
                                              int kvh, int pos, const int* tbl, int blk_lo,
                                              int nblk, int tid) {
  using Geo = ChunkGeo<D>;
  if (tid >= 2 * Geo::CPR) return;
  const int page = pos >> a.bs_shift;
  if (pos < 0 || page >= a.max_blk) {
    if (a.status && tid == 0) atomicOr(a.status, PKV_STATUS_SHORT_TABLE);
    return;
  }
  const int64_t phys = page >= blk_lo && page < blk_lo + nblk
                           ? tbl[page - blk_lo]
                           : a.block_tables[(int64_t)s * a.max_blk + page];
  if (phys <= 0 || phys >= a.num_blocks) {
    if (a.status && tid == 0) atomicOr(a.status, PKV_STATUS_BAD_BLOCK);
    return;
  }
  const bool is_v = tid >= Geo::CPR;
  const int64_t slot = (phys << a.bs_shift) + (pos & ((1 << a.bs_shift) - 1));
  char* pool = static_cast<char*>(const_cast<void*>(is_v ? a.v_pool : a.k_pool));
  const u32x4 piece = *reinterpret_cast<const u32x4*>(lds + tid * 16);
  if constexpr (KV8) {
    *reinterpret_cast<u32x2*>(pool + (slot * a.hkv + kvh) * D + (tid % Geo::CPR) * 8) =
        narrow8<T>(piece);
  } else {
    *reinterpret_cast<u32x4*>(pool + (slot * a.hkv + kvh) * D * 2 + (tid % Geo::CPR) * 16) =
        piece;
  }
}

// Block-wide exclusive scan of one int per thread (NW wavefronts); returns
// the total. Each wavefront scans its 64 values with lane shuffles, then the
// wavefront totals are combined through LDS (two barriers in all).
template <int NW>
__device__ __forceinline__ int block_scan(int x, int* sh, int& excl) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  int incl = x;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  if (lane == 63) sh[w] = incl;
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const int t = sh[i];
    before += i < w ? t : 0;
    total += t;
  }
  __syncthreads();  // sh is reused by the next scan
  excl = before + incl - x;
  // the same for every thread: keep it scalar
  return __builtin_amdgcn_readfirstlane(total);
}

// Q^T fragments of one (token, kv head): head 16*nt + l16, dims of piece
// 4*ks + grp.
template <typename T, int D, int NT>
__device__ __forceinline__ void load_q(typename Ops<T>::v8 (&qf)[NT][D / 32], const T* q,
                                       int64_t qrow0, int grp, int l16) {
  using v8 = typename Ops<T>::v8;
  const T* __restrict__ base = q + qrow0 * D;  // wavefront-uniform
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks)
      qf[nt][ks] = *reinterpret_cast<const v8*>(
          base + (unsigned)((16 * nt + l16) * D + (4 * ks + grp) * 8));
}

}  // namespace mfma
}  // namespace pkv
