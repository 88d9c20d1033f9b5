// Paged attention forward for gfx950: block-table gather fused with
// QK^T, online softmax and PV, split-K over the context with a merge pass.
//
// Semantics follow pagedattn.forward (kernels/pagedattn/pagedattn.cu:142-447):
//   kv_len = min(seq_lens[s], max_blk * bs)                       (:187-189)
//   ctx    = causal ? max(kv_len - q_len, 0) : 0                   (:196-200)
//   query i sees key j iff j < kv_len and (!causal or j <= ctx+i) (:315-329)
//   kv head = q head / (hq / hkv)                                  (:180)
//   rows with no visible key: out = 0, lse = +inf                  (:418-446)
// but nothing of its structure: there the grid is one CTA per (sequence,
// query head, 64-query tile), each re-streaming the whole context. Here a
// workgroup owns a tile of (query token, head) ROWS that share one kv head,
// so every K/V token is staged once per tile and reused by every query head
// of the group (for decode, one tile holds all heads of the group), and the
// context is cut into partitions that run as separate workgroups (split-K);
// a merge kernel combines the partial (max, sum, output) triples.
//
// Softmax runs in base 2: scores are scaled by scale*log2(e) and
// exponentiated with exp2, so the running max m and lse are converted back
// with ln(2) only at the end.
#include "pkv_internal.h"

#include <math.h>

namespace pkv {
namespace {

constexpr int kThreads = 256;
constexpr float kLn2 = 0.6931471805599453f;

template <typename T>
__device__ __forceinline__ float to_f32(T x) {
  return (float)x;
}
template <typename T>
__device__ __forceinline__ T from_f32(float x) {
  return (T)x;
}

// ---------------------------------------------------------------------------
// Generic kernel: any dtype, any group size, any q_len, d <= DMAX.
// 256 threads; thread t owns row t/8 and, within it, keys (t%8)+8e of each
// 32-key chunk for QK and output columns (t%8)+8j for PV. Row max / sum
// reductions are 8-lane shuffles inside one wavefront.
// ---------------------------------------------------------------------------
template <typename T, int DMAX>
__global__ __launch_bounds__(kThreads) void attn_rows_kernel(AttnArgs a) {
  constexpr int R = kGenRows;
  constexpr int C = kChunk;
  constexpr int DP = DMAX + 1;  // odd pitch: row-strided reads hit distinct banks
  constexpr int NJ = DMAX / 8;
  __shared__ float Qs[R][DP];
  __shared__ float Ks[C][DP];
  __shared__ float Vs[C][DP];
  __shared__ float Ps[R][C + 1];

  // sequence fastest: consecutive workgroups (round-robin over the XCDs)
  // belong to different sequences, so every XCD sees a share of the work
  const int tid = threadIdx.x;
  const int part = blockIdx.z;
  const int tile = blockIdx.y;
  const int s = blockIdx.x / a.hkv;
  const int kvh = blockIdx.x - s * a.hkv;
  TileGeom g;
  if (!tile_geom(a, s, tile, R, g)) return;
  if (part >= g.nparts) return;
  const int D = a.d;
  const int G = a.group;
  const int r0 = tile * R;
  const int kv_lo = part * g.part_len;
  const int kv_hi = min(kv_lo + g.part_len, g.kv_limit);

  const T* __restrict__ q = static_cast<const T*>(a.q);
  const T* __restrict__ kp = static_cast<const T*>(a.k_pool);
  const T* __restrict__ vp = static_cast<const T*>(a.v_pool);
  const int32_t* __restrict__ table = a.block_tables + (int64_t)s * a.max_blk;
  const int bs_mask = (1 << a.bs_shift) - 1;

  for (int idx = tid; idx < R * D; idx += kThreads) {
    const int r = idx / D;
    const int dd = idx - r * D;
    float v = 0.f;
    if (r < g.rows_here) {
      const int rg = r0 + r;
      const int i = rg / G;
      const int h = rg - i * G;
      const int64_t qrow = (int64_t)(g.q_begin + i) * a.hq + kvh * G + h;
      v = to_f32(q[qrow * D + dd]);
    }
    Qs[r][dd] = v;
  }

  const int r = tid >> 3;
  const int c8 = tid & 7;
  const bool row_valid = r < g.rows_here;
  int vis_hi = kv_hi;
  if (a.causal) vis_hi = min(vis_hi, g.ctx + (r0 + r) / G + 1);

  float m = -INFINITY, l = 0.f;
  float o[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) o[j] = 0.f;

  for (int c0 = kv_lo; c0 < kv_hi; c0 += C) {
    __syncthreads();
    for (int idx = tid; idx < C * D; idx += kThreads) {
      const int t = idx / D;
      const int dd = idx - t * D;
      const int pos = c0 + t;
      float kv_k = 0.f, kv_v = 0.f;
      if (pos < kv_hi) {
        const int64_t phys = table[pos >> a.bs_shift];
        if (phys >= 0 && phys < a.num_blocks) {
          const int64_t off =
              (((phys << a.bs_shift) + (pos & bs_mask)) * a.hkv + kvh) * D + dd;
          kv_k = to_f32(kp[off]);
          kv_v = to_f32(vp[off]);
        } else if (a.status && dd == 0) {
          atomicOr(a.status, PKV_STATUS_BAD_BLOCK);
        }
      }
      Ks[t][dd] = kv_k;
      Vs[t][dd] = kv_v;
    }
    __syncthreads();

    float sc[4];
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = c8 + 8 * e;
      float acc = 0.f;
      for (int dd = 0; dd < D; ++dd) acc = fmaf(Qs[r][dd], Ks[j][dd], acc);
      const bool vis = row_valid && (c0 + j) < vis_hi;
      sc[e] = vis ? acc * a.scale_log2 : -INFINITY;
      mx = fmaxf(mx, sc[e]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 1, 8));
    mx = fmaxf(mx, __shfl_xor(mx, 2, 8));
    mx = fmaxf(mx, __shfl_xor(mx, 4, 8));
    const float m_new = fmaxf(m, mx);
    const float ref = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m - ref);
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float p = exp2f(sc[e] - ref);
      Ps[r][c8 + 8 * e] = p;
      psum += p;
    }
    psum += __shfl_xor(psum, 1, 8);
    psum += __shfl_xor(psum, 2, 8);
    psum += __shfl_xor(psum, 4, 8);
    l = l * alpha + psum;
    m = m_new;
    __syncthreads();
#pragma unroll
    for (int jd = 0; jd < NJ; ++jd) {
      const int dd = c8 + 8 * jd;
      if (dd < D) {
        float acc = o[jd] * alpha;
        for (int j = 0; j < C; ++j) acc = fmaf(Ps[r][j], Vs[j][dd], acc);
        o[jd] = acc;
      }
    }
  }

  if (!row_valid) return;
  const int rg = r0 + r;
  const int i = rg / G;
  const int h = rg - i * G;
  const int64_t qrow = (int64_t)(g.q_begin + i) * a.hq + kvh * G + h;
  if (g.nparts == 1) {
    T* __restrict__ out = static_cast<T*>(a.out);
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int jd = 0; jd < NJ; ++jd) {
      const int dd = c8 + 8 * jd;
      if (dd < D) out[qrow * D + dd] = from_f32<T>(o[jd] * inv);
    }
    if (a.lse && c8 == 0) a.lse[qrow] = l > 0.f ? (m + log2f(l)) * kLn2 : INFINITY;
  } else {
    const int64_t unit =
        ((int64_t)blockIdx.x * a.tiles_max + tile) * a.parts_max + part;
    float* __restrict__ wo = a.ws_o + (unit * R + r) * D;
#pragma unroll
    for (int jd = 0; jd < NJ; ++jd) {
      const int dd = c8 + 8 * jd;
      if (dd < D) wo[dd] = o[jd];
    }
    if (c8 == 0) {
      a.ws_ml[(unit * R + r) * 2 + 0] = m;
      a.ws_ml[(unit * R + r) * 2 + 1] = l;
    }
  }
}

// ---------------------------------------------------------------------------
// Split-K merge: for every row of a tile that was split, combine the
// partitions' (m_p, l_p, o_p): M = max m_p, w_p = 2^(m_p - M),
// out = sum w_p o_p / sum w_p l_p, lse = (M + log2 sum w_p l_p) ln 2.
// Grid (n_seq * hkv, tiles, ceil(rows * d/4 / 256)); one thread per
// (row, 4 output columns).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kThreads) void merge_kernel(AttnArgs a,
                                                         int rows_per_tile) {
  const int tile = blockIdx.y;
  const int s = blockIdx.x / a.hkv;
  const int kvh = blockIdx.x - s * a.hkv;
  const int D = a.d;
  const int quads = D / 4;
  const int item = blockIdx.z * kThreads + threadIdx.x;
  const int r = item / quads;
  const int d0 = (item - r * quads) * 4;
  const int64_t unit0 = ((int64_t)blockIdx.x * a.tiles_max + tile) * a.parts_max;
  // One pass with a running max; the loads of kMB partitions are issued
  // before any is consumed and never sit under a branch (a branch join
  // would make the compiler wait for every load issued before it), so the
  // merge costs ceil(nparts / kMB) memory latencies. The first batch is
  // requested before the sequence's metadata: rows and partitions past the
  // ones that exist are read from the workspace (in bounds) and dropped.
  constexpr int kMB = 8;
  const int rr = min(r, rows_per_tile - 1);
  float mm[kMB], ll[kMB];
  float4 oo[kMB];
  auto load_batch = [&](int p0, int last) {
#pragma unroll
    for (int j = 0; j < kMB; ++j) {
      const int64_t row = (unit0 + min(p0 + j, last)) * rows_per_tile + rr;
      mm[j] = a.ws_ml[row * 2];
      ll[j] = a.ws_ml[row * 2 + 1];
      oo[j] = *reinterpret_cast<const float4*>(a.ws_o + row * D + d0);
    }
  };
  load_batch(0, a.parts_max - 1);
  TileGeom g;
  if (!tile_geom(a, s, tile, rows_per_tile, g)) return;
  if (g.nparts == 1) return;
  if (r >= g.rows_here) return;
  const int G = a.group;
  const int rg = tile * rows_per_tile + r;
  const int i = rg / G;
  const int h = rg - i * G;
  const int64_t qrow = (int64_t)(g.q_begin + i) * a.hq + kvh * G + h;
  T* __restrict__ out = static_cast<T*>(a.out) + qrow * D + d0;
  float M = -INFINITY;
  float L = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int p0 = 0; p0 < g.nparts; p0 += kMB) {
    if (p0 > 0) load_batch(p0, g.nparts - 1);
#pragma unroll
    for (int j = 0; j < kMB; ++j) {
      if (p0 + j >= g.nparts || mm[j] == -INFINITY) continue;
      const float Mn = fmaxf(M, mm[j]);
      const float sa = exp2f(M - Mn);
      const float sb = exp2f(mm[j] - Mn);
      L = L * sa + ll[j] * sb;
      acc.x = acc.x * sa + oo[j].x * sb;
      acc.y = acc.y * sa + oo[j].y * sb;
      acc.z = acc.z * sa + oo[j].z * sb;
      acc.w = acc.w * sa + oo[j].w * sb;
      M = Mn;
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  out[0] = from_f32<T>(acc.x * inv);
  out[1] = from_f32<T>(acc.y * inv);
  out[2] = from_f32<T>(acc.z * inv);
  out[3] = from_f32<T>(acc.w * inv);
  if (a.lse && d0 == 0) a.lse[qrow] = L > 0.f ? (M + log2f(L)) * kLn2 : INFINITY;
}

template <typename T>
int launch_merge(const AttnArgs& a, const AttnPlan& p, hipStream_t stream) {
  const int items = p.rows * (a.d / 4);
  hipLaunchKernelGGL((merge_kernel<T>),
                     dim3(a.n_seq * a.hkv, p.tiles_max, (items + kThreads - 1) / kThreads),
                     dim3(kThreads), 0, stream, a, p.rows);
  return check_launch("merge_kernel");
}

template <typename T>
int launch_generic(const AttnArgs& a, const AttnPlan& p, hipStream_t stream) {
  const dim3 grid(a.n_seq * a.hkv, p.tiles_max, p.parts_max);
  if (a.d <= 64) {
    hipLaunchKernelGGL((attn_rows_kernel<T, 64>), grid, dim3(kThreads), 0, stream, a);
  } else if (a.d <= 128) {
    hipLaunchKernelGGL((attn_rows_kernel<T, 128>), grid, dim3(kThreads), 0, stream, a);
  } else {
    hipLaunchKernelGGL((attn_rows_kernel<T, 256>), grid, dim3(kThreads), 0, stream, a);
  }
  int rc = check_launch("attn_rows_kernel");
  if (rc != PKV_OK || p.parts_max == 1) return rc;
  return launch_merge<T>(a, p, stream);
}

template <typename T>
int launch_mfma(const AttnArgs& a0, const AttnPlan& p, int dtype, hipStream_t stream) {
  AttnArgs a = a0;
  // split sequences merged inside the decode kernel when the workspace
  // header has a counter for every (sequence, kv head) pair
  if (p.parts_max > 1 && p.tiles_max == 1 && a.ws_o &&
      (int64_t)a.n_seq * a.hkv <= kMergeCtrMax)
    a.merge_ctr = reinterpret_cast<int*>(reinterpret_cast<char*>(a.ws_o) - kWsCounterBytes) +
                  kMergeCtrOff;
  int rc = launch_decode_mfma(a, p, dtype, stream);
  if (rc != PKV_OK || p.parts_max == 1 || a.merge_ctr) return rc;
  return launch_merge<T>(a, p, stream);
}

int ceil_div_h(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

}  // namespace

// Whether the persistent kernel takes this problem: one record per
// (sequence, kv head) pair fits the workspace's record region, and every
// table row has an entry (the kernel reads entry 0 of a row unconditionally).
bool sk_fits(int64_t virt, int max_blk) {
  return virt >= 1 && virt <= kMaxCounters && max_blk >= 1;
}


AttnPlan plan_attention(int n_seq, int max_q_len, int hq, int hkv, int d,
                        int max_blk, int block_size, int max_kv_len,
                        int part_tokens, int dtype) {
  AttnPlan p{};
  // fp8 pools are read by the MFMA kernels only (rows widened in LDS)
  const bool kv8 = dtype_kv8(dtype);
  dtype = dtype_base(dtype);
  const int group = hq / hkv;
  // the MFMA kernels read table entry 0 of a row unconditionally: with no
  // table (every context empty) the generic kernel writes the empty rows
  const bool mfma = decode_mfma_supported(dtype, max_q_len, group, d) && max_blk >= 1;
  const int64_t virt = (int64_t)n_seq * hkv;
  const int64_t cap_tokens = (int64_t)max_blk * block_size;
  const int64_t kv_bound = max_kv_len > 0 && max_kv_len < cap_tokens ? max_kv_len : cap_tokens;
  // automatic choice: long context bounds (where fixed-length partitions
  // leave the long sequences' workgroups running alone) take the persistent
  // kernel, which gives every workgroup the same share of the actual work
  const bool persistent = part_tokens == PKV_PART_PERSISTENT ||
                          part_tokens == PKV_PART_STATIC || part_tokens == PKV_PART_STREAM ||
                          (part_tokens == 0 && kv_bound >= kSkAutoKv);
  if (mfma && persistent && sk_fits(virt, max_blk)) {
    // persistent kernel: partials of at most two segments per workgroup
    p.kind = 2;
    p.ws = part_tokens == PKV_PART_STREAM;
    p.rows = group;
    p.tiles_max = 1;
    p.part_tokens = 0;
    p.parts_max = 1;
    p.ws_bytes = sk_workspace_bytes(group, d);
    return p;
  }
  if (max_q_len > 1 && max_blk >= 1 && prefill_mfma_supported(dtype, group, d)) {
    // MFMA prefill: one workgroup per pair of query-token tiles (t and
    // n - 1 - t of a sequence), whole causal range
    p.kind = 3;
    p.rows = 128;
    p.tiles_max = 1;
    p.part_tokens = 0;
    p.parts_max = 1;
    p.ws_bytes = 0;
    return p;
  }
  if (kv8 && !mfma) {
    p.kind = -1;  // unsupported: reported by launch_attention
    return p;
  }
  if (!mfma && max_blk >= 1 && decode_small_supported(dtype, max_q_len, group, d)) {
    // small groups: one workgroup per (sequence, kv head, partition) of at
    // least 256 tokens, longer bounds longer partitions so the longest
    // context splits into at most 8 partials, merged in the same launch
    p.kind = 4;
    p.rows = group;
    p.tiles_max = 1;
    int plen = part_tokens > 0 ? part_tokens : 256;
    if (part_tokens <= 0)
      while (plen < 8192 && (int64_t)plen * 8 < kv_bound) plen *= 2;
    plen = (plen + kChunk - 1) / kChunk * kChunk;
    p.part_tokens = plen;
    p.parts_max = ceil_div_h(kv_bound > 0 ? kv_bound : 1, plen);
    if (p.parts_max < 1) p.parts_max = 1;
    // split sequences are merged in the kernel: every (sequence, kv head)
    // pair needs a counter of the workspace header
    if (p.parts_max > 1 && virt > kMergeCtrMax) {
      p.parts_max = 1;
      p.part_tokens = (int)((kv_bound + kChunk - 1) / kChunk * kChunk);
    }
    p.ws_bytes = p.parts_max > 1
                     ? kWsCounterBytes + (size_t)virt * p.parts_max * group * ((size_t)d + 2) *
                                             sizeof(float)
                     : 0;
    return p;
  }
  p.kind = mfma ? 1 : 0;
  p.rows = mfma ? group : kGenRows;
  p.tiles_max = ceil_div_h((int64_t)max_q_len * group, p.rows);
  if (p.tiles_max < 1) p.tiles_max = 1;
  const int64_t cap = (int64_t)max_blk * block_size;
  int64_t kvb = max_kv_len > 0 && max_kv_len < cap ? max_kv_len : cap;
  if (kvb < 1) kvb = 1;
  const int64_t units = (int64_t)n_seq * hkv * p.tiles_max;
  int plen = part_tokens;
  if (plen <= 0 && mfma) {
    // at least 4 wavefronts x 4 chunks of 32 tokens, to amortise the
    // workgroup prologue (table slice, Q) and keep loads pipelined; longer
    // bounds get longer partitions so the longest context splits into at
    // most 8 partials (merge work and partial traffic stay bounded)
    plen = 512;
    while (plen < 4096 && (int64_t)plen * 8 < kvb) plen *= 2;
  } else if (plen <= 0) {
    // Aim for ~2048 workgroups so the 256 CUs stay busy even when most
    // sequences are far below the bound.
    int64_t parts_target = (2048 + units - 1) / (units > 0 ? units : 1);
    if (parts_target < 1) parts_target = 1;
    plen = (int)((kvb + parts_target - 1) / parts_target);
    if (plen < 64) plen = 64;
  }
  plen = (plen + kChunk - 1) / kChunk * kChunk;
  p.part_tokens = plen;
  p.parts_max = ceil_div_h(kvb, plen);
  if (p.parts_max < 1) p.parts_max = 1;
  p.ws_bytes = p.parts_max > 1
                   ? kWsCounterBytes + (size_t)units * p.parts_max * p.rows *
                                           ((size_t)d + 2) * sizeof(float)
                   : 0;
  return p;
}

AttnSplit plan_split(int n_seq, int max_q_len, int hq, int hkv, int d, int max_blk,
                     int block_size, int max_kv_len, int part_tokens, int dtype,
                     bool has_qloc) {
  AttnSplit sp{};
  sp.mixed = has_qloc && max_q_len > 1 && n_seq >= 2 && max_blk >= 1 &&
             decode_mfma_supported(dtype_base(dtype), 1, hq / hkv, d);
  if (!sp.mixed) {
    sp.dec = plan_attention(n_seq, max_q_len, hq, hkv, d, max_blk, block_size, max_kv_len,
                            part_tokens, dtype);
    sp.ws_bytes = sp.dec.ws_bytes;
    return sp;
  }
  sp.dec = plan_attention(n_seq, 1, hq, hkv, d, max_blk, block_size, max_kv_len, part_tokens,
                          dtype);
  sp.pre = plan_attention(n_seq, max_q_len, hq, hkv, d, max_blk, block_size, max_kv_len,
                          part_tokens, dtype);
  sp.ws_bytes = sp.dec.ws_bytes > sp.pre.ws_bytes ? sp.dec.ws_bytes : sp.pre.ws_bytes;
  return sp;
}

int device_cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

SkArgs sk_args_for(const AttnArgs& a) {
  SkArgs k{};
  k.n_wg = 2 * device_cu_count() < kSkMaxWg ? 2 * device_cu_count() : kSkMaxWg;
  k.seg_cost = kSkSegCost;
  char* ws = reinterpret_cast<char*>(a.ws_o) - kWsCounterBytes;
  k.recs = reinterpret_cast<int4*>(ws + kWsCtrBytes);
  k.part_o = reinterpret_cast<uint16_t*>(a.ws_o);
  k.part_ml = reinterpret_cast<float*>(k.part_o + (size_t)kSkMaxWg * 2 * a.group * a.d);
  return k;
}

int launch_attention_mixed(const AttnArgs& ad, const AttnArgs& ap, int dtype,
                           hipStream_t stream) {
  if (ad.n_seq == 0) return PKV_OK;
  return launch_mixed_sk(ad, sk_args_for(ad), ap, dtype, stream);
}

int launch_attention(const AttnArgs& a, const AttnPlan& p, int dtype,
                     hipStream_t stream) {
  if (a.n_seq == 0) return PKV_OK;
  if (p.kind < 0)
    return fail(PKV_ERR_UNSUPPORTED,
                "fp8 KV pools need bf16/f16 queries, 16 or 32 query heads per kv head and "
                "head dim 64 or 128 (got group %d, d %d)", a.group, a.d);
  if (p.parts_max > 65535 || p.tiles_max > 65535)
    return fail(PKV_ERR_UNSUPPORTED, "attention grid too large (%d parts, %d tiles, %d seq*hkv)",
                p.parts_max, p.tiles_max, a.n_seq * a.hkv);
  if (p.kind == 2) {
    if (p.ws && decode_ws_supported(a, dtype))
      return launch_decode_ws(a, sk_args_for(a), dtype, stream);
    return launch_decode_sk(a, sk_args_for(a), dtype, stream);
  }
  if (p.kind == 1) {
    if (dtype == PKV_DTYPE_BF16) return launch_mfma<bf16>(a, p, dtype, stream);
    return launch_mfma<f16>(a, p, dtype, stream);
  }
  if (p.kind == 3) return launch_prefill_mfma(a, dtype, stream);
  if (p.kind == 4) {
    AttnArgs as = a;
    if (p.parts_max > 1 && a.ws_o)
      as.merge_ctr = reinterpret_cast<int*>(reinterpret_cast<char*>(a.ws_o) - kWsCounterBytes) +
                     kMergeCtrOff;
    return launch_decode_small(as, p, dtype, stream);
  }
  switch (dtype) {
    case PKV_DTYPE_F32: return launch_generic<float>(a, p, stream);
    case PKV_DTYPE_F16: return launch_generic<f16>(a, p, stream);
    case PKV_DTYPE_BF16: return launch_generic<bf16>(a, p, stream);
  }
  return fail(PKV_ERR_INVALID, "unknown dtype %d", dtype);
}

}  // namespace pkv
