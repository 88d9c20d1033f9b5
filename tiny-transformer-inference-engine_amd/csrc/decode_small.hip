// Paged decode for small query-head groups: G = hq / hkv in {1, 2, 4, 8}
// query heads per kv head, head dim 32, 64 or 128, fp32 / bf16 / fp16
// storage with fp32 arithmetic, one query token per sequence. These are the
// shapes the MFMA decode kernels do not take (their tiles are 16 heads
// tall): configs 1 and 2 of the benchmark (G 4 and 8, d 32). Same semantics
// as pagedattn.forward (kernels/pagedattn/pagedattn.cu:142-447) for
// q_len = 1.
//
// A workgroup of 4 wavefronts owns one (sequence, kv head, partition) and
// G of the group's query heads: a small batch splits each group's heads
// over several workgroups (they read the same K / V rows, and no merge is
// needed), so that the grid fills the CUs. A
// token row (D elements) is split into 16-byte pieces, one per lane, so a
// wavefront covers 64 / LPT tokens per step (LPT = lanes per row) and
// every lane issues one 16-byte load for K and one for V per token, four
// steps in flight (the 256 tokens of a planned partition in one round). Each lane holds the G query heads' elements of its
// piece, pre-scaled by softmax_scale * log2(e); a token's partial dot
// products are summed over its LPT lanes with DPP / cross-row swaps (VALU
// data movement). Every lane group keeps an online softmax (max, sum, O
// piece) per head over its tokens; at the end every group's state goes to
// LDS, each head's weights 2^(m - M) are formed once, and each output
// column is one weighted sum over the groups (a fold through lane
// exchanges, 4 levels of 8 heads x 10 values at bf16 d 32, took 3.5 us).
// A sequence split into several partitions is merged in the same launch
// by the last partition to finish (arrival counter, as in the partition
// decode kernel): no second launch. With the fused append (a.new_pos) the
// step's new row is taken from k_new / v_new at its position and written
// into the pool by the sequence's last partition.
#include "pkv_internal.h"

namespace pkv {
namespace {

constexpr int kSmThreads = 256;
constexpr int kSmWaves = kSmThreads / 64;
constexpr int kSmTblCap = 1024;    // table entries of a partition staged in LDS
constexpr int64_t kSmallGridTarget = 256;  // workgroups a launch aims for (one per CU)
constexpr float kSmLn2 = 0.69314718055994530942f;

template <typename T, int D, int G>
struct SmallGeo {
  static constexpr int E = 16 / (int)sizeof(T);  // elements per 16-byte piece
  static constexpr int LPT = D / E;              // lanes per token row
  static constexpr int TPW = 64 / LPT;           // tokens per wavefront step
  static_assert(LPT >= 1 && LPT <= 64 && (LPT & (LPT - 1)) == 0, "row pieces");
  // wavefront steps (tokens per lane group) in flight: a planned partition
  // of 256 tokens in one round, within the register budget (fewer heads,
  // fewer registers per token)
  static constexpr int STEPS_WANT = 256 / (4 * TPW);
  static constexpr int STEPS_CAP = G <= 2 ? 8 : 4;
  static constexpr int STEPS = STEPS_WANT < 1 ? 1 : (STEPS_WANT > STEPS_CAP ? STEPS_CAP : STEPS_WANT);
};

template <typename T, int E>
__device__ __forceinline__ void widen(const uint4& raw, float (&x)[E]) {
  T e[E];
  __builtin_memcpy(e, &raw, 16);
#pragma unroll
  for (int i = 0; i < E; ++i) x[i] = (float)e[i];
}

// Sum over the lanes lane ^ 1 .. lane ^ (N / 2) (a group of N lanes).
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += lane_xor<1>(x);
  if constexpr (N >= 4) x += lane_xor<2>(x);
  if constexpr (N >= 8) x += lane_xor<4>(x);
  if constexpr (N >= 16) x += lane_xor<8>(x);
  if constexpr (N >= 32) x += lane_xor<16>(x);
  if constexpr (N >= 64) x += lane_xor<32>(x);
  return x;
}

// Online-softmax state of one head: running max (log2 units), sum, and the
// lane's E output elements (unnormalised).
template <int E>
struct HeadState {
  float m, l;
  float o[E];
};

// 2^x by the bare v_exp_f32 (the library exp2f adds a rescaling for results
// below 2^-126: weights that vanish next to the running maximum's 1).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Folds state b into a (both over disjoint token sets), branch-free: a side
// that has seen no key (max -inf) gets weight 2^-inf = 0, and when neither
// has, the reference point 0 keeps the weights 0 rather than NaN.
template <int E>
__device__ __forceinline__ void combine(HeadState<E>& a, float bm, float bl, const float (&bo)[E]) {
  const float M = fmaxf(a.m, bm);
  const float ref = M == -INFINITY ? 0.f : M;
  const float wa = fast_exp2(a.m - ref);
  const float wb = fast_exp2(bm - ref);
  a.l = a.l * wa + bl * wb;
#pragma unroll
  for (int i = 0; i < E; ++i) a.o[i] = fmaf(a.o[i], wa, bo[i] * wb);
  a.m = M;
}

template <typename T, int E>
__device__ __forceinline__ void store_piece(T* dst, const float (&x)[E], float s) {
  T v[E];
#pragma unroll
  for (int i = 0; i < E; ++i) v[i] = (T)(x[i] * s);
  uint4 raw;
  __builtin_memcpy(&raw, v, 16);
  *reinterpret_cast<uint4*>(dst) = raw;
}

template <typename T, int D, int G>
__global__ __launch_bounds__(kSmThreads) void decode_small_kernel(AttnArgs a) {
  using Geo = SmallGeo<T, D, G>;
  constexpr int E = Geo::E, LPT = Geo::LPT, TPW = Geo::TPW;
  constexpr int kSmSteps = Geo::STEPS;
  constexpr int WG_STEP = kSmWaves * TPW;  // tokens of one workgroup step
  // the final combination: s_o holds column d of head h for lane group gi
  // at (h D + d) OP + gi (OP = NG + pad, so that the pieces of one
  // wavefront's stores fall on distinct banks)
  constexpr int NG = kSmWaves * TPW;  // lane groups of the workgroup
  constexpr int OP = NG + (TPW / E > 1 ? TPW / E : 1);
  static_assert(NG <= 64 && G * 32 <= kSmThreads, "one lane pair per group, 32 lanes per head");
  __shared__ int tbl[kSmTblCap];
  __shared__ float s_o[G * D * OP];
  __shared__ float s_m[G][NG], s_l[G][NG], s_w[G][NG];
  __shared__ float s_M[G], s_L[G];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int piece = lane % LPT;
  const int tg = lane / LPT;
  const int part = blockIdx.y;
  // blockIdx.x = hs * (n_seq * hkv) + (s * hkv + kvh): head slice hs of the
  // group (G of its a.group heads); the slices of one (sequence, kv head)
  // are n_seq * hkv apart, so they share an XCD (and its L2) whenever that
  // count is a multiple of 8
  const int nsv = a.n_seq * a.hkv;
  const int hs = blockIdx.x / nsv;
  const int sv = blockIdx.x - hs * nsv;
  const int s = sv / a.hkv;
  const int kvh = sv - s * a.hkv;
  const int h0 = kvh * a.group + hs * G;  // the slice's first query head

  // Requested before the sequence's metadata arrives (one round trip
  // instead of three): the partition's first table entries at the planned
  // partition length (one per thread, clamped to the row) and the Q rows of
  // query token s (a decode batch's query_start_loc is 0, 1, 2, ...; when it
  // is not, the rows are requested again once it has arrived).
  const int32_t* table = a.block_tables + (int64_t)s * a.max_blk;
  const int spec_blk0 = (part * a.part_tokens) >> a.bs_shift;
  const int tspec = table[max(0, min(spec_blk0 + tid, a.max_blk - 1))];
  // fused append: the sequence's new row goes to position new_pos[s]; the
  // partition holding that position takes it from k_new / v_new (the pool
  // does not hold it yet) and the last partition writes it into the pool
  const int npos = a.new_pos ? a.new_pos[s] : -1;
  uint4 qraw[G];
  if (s < a.n_tokens) {  // uniform
    const T* qp = static_cast<const T*>(a.q) + ((int64_t)s * a.hq + h0) * D + piece * E;
#pragma unroll
    for (int h = 0; h < G; ++h) qraw[h] = *reinterpret_cast<const uint4*>(qp + (int64_t)h * D);
  }
  TileGeom g;
  if (!tile_geom(a, s, 0, G, g)) return;
  if (part >= g.nparts) return;
  const int kv_lo = part * g.part_len;
  const int kv_hi = min(kv_lo + g.part_len, g.kv_limit);
  const int64_t qrow0 = (int64_t)g.q_begin * a.hq + h0;
  if (g.q_begin != s) {  // uniform
    const T* qp = static_cast<const T*>(a.q) + qrow0 * D + piece * E;
#pragma unroll
    for (int h = 0; h < G; ++h) qraw[h] = *reinterpret_cast<const uint4*>(qp + (int64_t)h * D);
  }
  // the speculative entries are this partition's first window unless the
  // sequence outgrew the planned bound (longer partitions)
  const bool spec_ok = g.part_len == a.part_tokens;

  // Q of the group, this lane's piece, scaled to log2 units
  float q[G][E];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    widen<T, E>(qraw[h], q[h]);
#pragma unroll
    for (int i = 0; i < E; ++i) q[h][i] *= a.scale_log2;
  }
  HeadState<E> st[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    st[h].m = -INFINITY;
    st[h].l = 0.f;
#pragma unroll
    for (int i = 0; i < E; ++i) st[h].o[i] = 0.f;
  }

  const char* kbase = static_cast<const char*>(a.k_pool);
  const char* vbase = static_cast<const char*>(a.v_pool);
  // the new row's pieces (query token q_begin of the sequence)
  const int64_t new_off = (((int64_t)g.q_begin * a.hkv + kvh) * D + piece * E) * sizeof(T);
  const char* knew = a.new_pos ? static_cast<const char*>(a.k_new) + new_off : nullptr;
  const char* vnew = a.new_pos ? static_cast<const char*>(a.v_new) + new_off : nullptr;
  const int64_t row_bytes = (int64_t)a.hkv * D * sizeof(T);
  const int64_t piece_off = ((int64_t)kvh * D + piece * E) * sizeof(T);
  const int bmask = (1 << a.bs_shift) - 1;
  bool bad = false;
  // the partition in windows whose table entries fit the LDS table (one
  // window unless a sequence outgrew the planned bound)
  const int win = (kSmTblCap - 1) << a.bs_shift;
  for (int lo = kv_lo; lo < kv_hi; lo += win) {
  const int hi = min(lo + win, kv_hi);
  const int blk_lo = lo >> a.bs_shift;
  const int nblk = ((hi - 1) >> a.bs_shift) + 1 - blk_lo;
  __syncthreads();  // the previous window's entries are no longer read
  if (spec_ok && lo == kv_lo && nblk <= kSmThreads) {
    if (tid < nblk) tbl[tid] = tspec;
  } else {
    for (int i = tid; i < nblk; i += kSmThreads) tbl[i] = table[blk_lo + i];
  }
  __syncthreads();
  for (int t0 = lo + w * TPW + tg; t0 < hi; t0 += WG_STEP * kSmSteps) {
    // the loads of kSmSteps tokens, unconditional (tokens past the window
    // read its last token; their scores are masked)
    // (a table entry outside the pool reads block 0, then counts as zeros)
    uint4 kr[kSmSteps], vr[kSmSteps];
    bool okb[kSmSteps];
#pragma unroll
    for (int j = 0; j < kSmSteps; ++j) {
      const int t = min(t0 + j * WG_STEP, hi - 1);
      const int blk = tbl[(t >> a.bs_shift) - blk_lo];
      okb[j] = blk >= 0 && blk < a.num_blocks;
      bad |= !okb[j];
      const int64_t off =
          ((int64_t)(okb[j] ? blk : 0) * (bmask + 1) + (t & bmask)) * row_bytes + piece_off;
      const bool isnew = t == npos;  // npos >= 0 only with the fused append
      okb[j] = okb[j] || isnew;
      kr[j] = *reinterpret_cast<const uint4*>(isnew ? knew : kbase + off);
      vr[j] = *reinterpret_cast<const uint4*>(isnew ? vnew : vbase + off);
    }
#pragma unroll
    for (int j = 0; j < kSmSteps; ++j) {
      const bool valid = t0 + j * WG_STEP < hi;
      float k[E], v[E];
      widen<T, E>(kr[j], k);
      widen<T, E>(vr[j], v);
#pragma unroll
      for (int i = 0; i < E; ++i) {
        k[i] = okb[j] ? k[i] : 0.f;
        v[i] = okb[j] ? v[i] : 0.f;
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < E; ++i) dot = fmaf(q[h][i], k[i], dot);
        dot = group_sum<LPT>(dot);
        // a masked token: score -inf, weight 0, the state unchanged
        const float sc = valid ? dot : -INFINITY;
        const float mn = fmaxf(st[h].m, sc);
        const float ref = mn == -INFINITY ? 0.f : mn;
        const float alpha = fast_exp2(st[h].m - ref);  // m = -inf: 0
        const float p = fast_exp2(sc - ref);
        st[h].l = fmaf(st[h].l, alpha, p);
#pragma unroll
        for (int i = 0; i < E; ++i) st[h].o[i] = fmaf(p, v[i], st[h].o[i] * alpha);
        st[h].m = mn;
      }
    }
  }
  }
  if (bad && a.status) atomicOr(a.status, PKV_STATUS_BAD_BLOCK);

  // fused append: the last partition writes the new row into its pool slot,
  // after the table and pool checks of the stand-alone append (status bits
  // instead of the write); threads [0, LPT) the K pieces, [LPT, 2 LPT) V
  if (a.new_pos && part == g.nparts - 1 && hs == 0 && tid < 2 * LPT) {
    const int page = npos >> a.bs_shift;
    if (npos < 0 || page >= a.max_blk) {
      if (a.status && tid == 0) atomicOr(a.status, PKV_STATUS_SHORT_TABLE);
    } else {
      const int64_t phys = table[page];
      if (phys <= 0 || phys >= a.num_blocks) {
        if (a.status && tid == 0) atomicOr(a.status, PKV_STATUS_BAD_BLOCK);
      } else {
        const bool is_v = tid >= LPT;
        const int pc = tid % LPT;
        const int64_t slot = (phys << a.bs_shift) + (npos & bmask);
        const int64_t src = (((int64_t)g.q_begin * a.hkv + kvh) * D + pc * E) * sizeof(T);
        const int64_t dst = ((slot * a.hkv + kvh) * D + pc * E) * sizeof(T);
        const uint4 x = *reinterpret_cast<const uint4*>(
            static_cast<const char*>(is_v ? a.v_new : a.k_new) + src);
        *reinterpret_cast<uint4*>(static_cast<char*>(const_cast<void*>(is_v ? a.v_pool : a.k_pool)) +
                                  dst) = x;
      }
    }
  }

  // ---- combine: every lane group's state through LDS; per head the
  // reference M (the groups' largest max) and each group's weight
  // 2^(m - M) once (32 lanes per head, two groups per lane), then per pair
  // of output columns one weighted sum over the groups, in group order ----
  {
    const int gi = w * TPW + tg;
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int i = 0; i < E; ++i) s_o[(h * D + piece * E + i) * OP + gi] = st[h].o[i];
      if (piece == 0) {
        s_m[h][gi] = st[h].m;
        s_l[h][gi] = st[h].l;
      }
    }
  }
  __syncthreads();
  if (tid < 32 * G) {
    const int h = tid >> 5, j = tid & 31;
    const bool ha = j < NG, hb = j + 32 < NG;
    const float ma = ha ? s_m[h][j] : -INFINITY;
    const float mb = hb ? s_m[h][j + 32] : -INFINITY;
    float M = fmaxf(ma, mb);
    M = fmaxf(M, lane_xor<1>(M));
    M = fmaxf(M, lane_xor<2>(M));
    M = fmaxf(M, lane_xor<4>(M));
    M = fmaxf(M, lane_xor<8>(M));
    M = fmaxf(M, lane_xor<16>(M));
    const float ref = M == -INFINITY ? 0.f : M;  // no key seen: weights 0, not NaN
    const float wa = fast_exp2(ma - ref), wb = fast_exp2(mb - ref);
    if (ha) s_w[h][j] = wa;
    if (hb) s_w[h][j + 32] = wb;
    float L = (ha ? s_l[h][j] * wa : 0.f) + (hb ? s_l[h][j + 32] * wb : 0.f);
    L += lane_xor<1>(L);
    L += lane_xor<2>(L);
    L += lane_xor<4>(L);
    L += lane_xor<8>(L);
    L += lane_xor<16>(L);
    if (j == 0) {
      s_M[h] = M;
      s_L[h] = L;
    }
  }
  __syncthreads();
  T* out = static_cast<T*>(a.out);
  const bool split = g.nparts > 1;
  const int64_t unit = (int64_t)blockIdx.x * a.parts_max + part;
  for (int pi = tid; pi < G * D / 2; pi += kSmThreads) {
    const int h = pi / (D / 2);
    const int d = 2 * (pi - h * (D / 2));
    const float* o0 = s_o + (h * D + d) * OP;
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll 8
    for (int gg = 0; gg < NG; ++gg) {
      const float wg = s_w[h][gg];
      acc0 = fmaf(o0[gg], wg, acc0);
      acc1 = fmaf(o0[OP + gg], wg, acc1);
    }
    const float L = s_L[h];
    const float inv = L > 0.f ? 1.f / L : 0.f;
    if (!split) {
      const T pr[2] = {(T)(acc0 * inv), (T)(acc1 * inv)};
      __builtin_memcpy(out + (qrow0 + h) * D + d, pr, sizeof(pr));
      if (d == 0 && a.lse) a.lse[qrow0 + h] = L > 0.f ? (s_M[h] + log2f(L)) * kSmLn2 : INFINITY;
    } else {
      // split-K partial: O / sum in fp32 and (max, sum), written through to
      // memory for the partition that completes the sequence's count
      const float2 pr = make_float2(acc0 * inv, acc1 * inv);
      uint64_t b;
      __builtin_memcpy(&b, &pr, 8);
      st_agent64(a.ws_o + (unit * G + h) * D + d, b);
      if (d == 0) {
        const float2 ml = make_float2(s_M[h], L);
        __builtin_memcpy(&b, &ml, 8);
        st_agent64(a.ws_ml + (unit * G + h) * 2, b);
      }
    }
  }
  if (!split) return;
  // thread (h, pc) of the first G * LPT threads merges head h's piece pc
  const bool owner = tid < G * LPT;
  const int oh = tid / LPT;
  const int opc = tid - oh * LPT;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    int* ctr = a.merge_ctr + blockIdx.x;
    const int old = fetch_add_agent(ctr, 1);
    s_last = old == g.nparts - 1;
    if (s_last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((old < 0 || old >= g.nparts) && a.status) atomicOr(a.status, PKV_STATUS_DIRTY_WORKSPACE);
  }
  __syncthreads();
  if (!s_last || !owner) return;
  // every partial in partition order (the result does not depend on which
  // partition arrives last); device-coherent loads: the partials were
  // written through from other XCDs during this launch
  HeadState<E> mg;
  mg.m = -INFINITY;
  mg.l = 0.f;
#pragma unroll
  for (int i = 0; i < E; ++i) mg.o[i] = 0.f;
  const int64_t unit0 = (int64_t)blockIdx.x * a.parts_max;
  for (int p = 0; p < g.nparts; ++p) {
    const int64_t row = (unit0 + p) * G + oh;
    const uint64_t mlb = __hip_atomic_load(reinterpret_cast<const uint64_t*>(a.ws_ml + row * 2),
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float2 ml;
    __builtin_memcpy(&ml, &mlb, 8);
    float bo[E];
#pragma unroll
    for (int i = 0; i < E; i += 2) {
      const uint64_t ob = __hip_atomic_load(
          reinterpret_cast<const uint64_t*>(a.ws_o + row * D + opc * E + i), __ATOMIC_RELAXED,
          __HIP_MEMORY_SCOPE_AGENT);
      float2 pr;
      __builtin_memcpy(&pr, &ob, 8);
      bo[i] = pr.x * ml.y;  // back to unnormalised
      bo[i + 1] = pr.y * ml.y;
    }
    combine(mg, ml.x, ml.y, bo);
  }
  const float inv = mg.l > 0.f ? 1.f / mg.l : 0.f;
  store_piece<T, E>(out + (qrow0 + oh) * D + opc * E, mg.o, inv);
  if (opc == 0 && a.lse) a.lse[qrow0 + oh] = mg.l > 0.f ? (mg.m + log2f(mg.l)) * kSmLn2 : INFINITY;
}

template <typename T, int D>
int launch_small_d(const AttnArgs& a, int heads, dim3 grid, hipStream_t stream) {
  switch (heads) {
    case 1: hipLaunchKernelGGL((decode_small_kernel<T, D, 1>), grid, dim3(kSmThreads), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((decode_small_kernel<T, D, 2>), grid, dim3(kSmThreads), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((decode_small_kernel<T, D, 4>), grid, dim3(kSmThreads), 0, stream, a); break;
    default: hipLaunchKernelGGL((decode_small_kernel<T, D, 8>), grid, dim3(kSmThreads), 0, stream, a); break;
  }
  return check_launch("decode_small_kernel");
}

template <typename T>
int launch_small_t(const AttnArgs& a, int heads, dim3 grid, hipStream_t stream) {
  if (a.d == 32) return launch_small_d<T, 32>(a, heads, grid, stream);
  if (a.d == 64) return launch_small_d<T, 64>(a, heads, grid, stream);
  return launch_small_d<T, 128>(a, heads, grid, stream);
}

}  // namespace

bool decode_small_supported(int dtype, int max_q_len, int group, int d) {
  return max_q_len == 1 && (group == 1 || group == 2 || group == 4 || group == 8) &&
         (d == 32 || d == 64 || d == 128) &&
         (dtype == PKV_DTYPE_F32 || dtype == PKV_DTYPE_BF16 || dtype == PKV_DTYPE_F16);
}

int launch_decode_small(const AttnArgs& a, const AttnPlan& p, int dtype, hipStream_t stream) {
  if (p.parts_max > 1 && !a.merge_ctr)
    return fail(PKV_ERR_WORKSPACE, "decode_small: split partitions need the workspace counters");
  // a small batch splits each group's heads over several workgroups (each
  // reads the same K / V rows and owns some heads: no merge), until the
  // grid has about one workgroup per CU
  const int64_t nsv = (int64_t)a.n_seq * a.hkv;
  int hsplit = 1;
  while (hsplit < a.group && nsv * p.parts_max * hsplit < kSmallGridTarget &&
         (p.parts_max == 1 || nsv * hsplit * 2 <= kMergeCtrMax))
    hsplit *= 2;
  if (nsv * hsplit > 0x7fffffff)
    return fail(PKV_ERR_UNSUPPORTED, "decode_small: grid too large");
  const dim3 grid((unsigned)(nsv * hsplit), p.parts_max);
  const int heads = a.group / hsplit;
  if (dtype == PKV_DTYPE_F32) return launch_small_t<float>(a, heads, grid, stream);
  if (dtype == PKV_DTYPE_BF16) return launch_small_t<bf16>(a, heads, grid, stream);
  return launch_small_t<f16>(a, heads, grid, stream);
}

}  // namespace pkv
