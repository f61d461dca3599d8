// Deterministic token-choice top-k SwiGLU mixture of experts.
//   act = SwiGLU(x . gate_e^T, x . up_e^T)   (one fused GEMM launch)
//   y   = act . down_e^T                     (one GEMM launch)
//   out[t] = fixed left-to-right sum over the top-k slots of round(y(t, s) * round(w[t,s]))
// Dense path (biops_moe): every expert for every token, y[e, t] for all (e, t).
// Sparse path (biops_moe_sparse): the routes r = t*k + s are packed by expert into consecutive
// rows (a row -> token table; the GEMM reads x rows through it) and each expert multiplies only
// its own rows (grouped GEMMs).  Every GEMM output row is
// computed by the same fixed MFMA sequence whatever the other rows of its launch are, so the
// sparse y row of route (t, s) has the bits of the dense y[sel[t,s], t] and both paths give
// identical outputs.
// No atomics anywhere: route ranks come from wavefront ballots, and every output element is
// written by exactly one thread.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "gemm.h"

namespace biops {

struct CombineArgs {
  const void* y;          // dense: [E, T, D]; sparse: packed rows [R, D]
  const void* w;          // [T, k]
  const int64_t* sel;     // [T, k]
  const int32_t* route_row;  // sparse: packed y row of route t*k+s; nullptr for dense
  void* out;              // [T, D]
  int32_t* bad;           // optional error flag
  int64_t T, D, E, k;
  int w_dtype;
  int32_t vec;
};

template <typename T>
__device__ __forceinline__ float load_weight(const void* w, int wdt, int64_t idx) {
  switch (wdt) {
    case BIOPS_F32: return Num<T>::round(reinterpret_cast<const float*>(w)[idx]);
    case BIOPS_F16: return Num<T>::round(Num<f16_t>::load(reinterpret_cast<const f16_t*>(w) + idx));
    default: return Num<T>::round(Num<bf16_t>::load(reinterpret_cast<const bf16_t*>(w) + idx));
  }
}

// Element e of a 16-byte chunk of T as fp32, and the reverse (chunk_put fills e in order).
template <typename T>
__device__ __forceinline__ float chunk_elem(const u32x4_t& v, int e) {
  if constexpr (sizeof(T) == 4) return __uint_as_float(v[e]);
  else return Num<T>::from_bits((v[e >> 1] >> (16 * (e & 1))) & 0xffffu);
}
template <typename T>
__device__ __forceinline__ void chunk_put(u32x4_t& v, int e, float x) {
  if constexpr (sizeof(T) == 4) {
    v[e] = __float_as_uint(x);
  } else {
    const uint32_t b = Num<T>::to_bits(x);
    v[e >> 1] = (e & 1) ? (v[e >> 1] | (b << 16)) : b;
  }
}

// One workgroup per token.  Vector path (16-byte rows): each thread owns one 16-byte column
// chunk per pass and keeps the y loads of 8 slots in flight before adding them in slot order;
// otherwise 4 scalar columns per thread.  Same arithmetic either way:
//   acc = v_0, acc = round(acc + v_s) for s = 1..k-1, v_s = round(y_s * round(w_s)).
template <typename T>
__global__ __launch_bounds__(256) void moe_combine_kernel(CombineArgs a) {
  constexpr int V = 16 / (int)sizeof(T);
  constexpr int G = 8;
  const int64_t t = blockIdx.x;
  // Every slot's index must be valid (the sparse path marks invalid ones with route row -1);
  // the checks load G slots at a time, so that their latencies overlap.  The y rows and
  // routing weights of the first G slots (every slot for k <= G) are kept for the sums below,
  // together with those loads.
  bool ok = true;
  int64_t row0[G];
  float w0[G];
  for (int64_t s0 = 0; s0 < a.k; s0 += G) {
    int64_t v[G];
    float wv[G];
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const int64_t r = t * a.k + s0 + u;
      v[u] = s0 + u < a.k ? (a.route_row ? (int64_t)a.route_row[r] : a.sel[r]) : 0;
      wv[u] = s0 + u < a.k ? load_weight<T>(a.w, a.w_dtype, r) : 0.f;
    }
#pragma unroll
    for (int u = 0; u < G; ++u) ok = ok && (a.route_row ? v[u] >= 0 : (v[u] >= 0 && v[u] < a.E));
    if (s0 == 0) {
#pragma unroll
      for (int u = 0; u < G; ++u) {
        // (an out-of-range index is never used: it clears ok)
        row0[u] = a.route_row ? v[u] : (v[u] >= 0 && v[u] < a.E ? v[u] * a.T + t : 0);
        w0[u] = wv[u];
      }
    }
  }
  if (!ok && threadIdx.x == 0 && a.bad) *a.bad = 1;
  T* out = reinterpret_cast<T*>(a.out) + t * a.D;
  const T* ybase = reinterpret_cast<const T*>(a.y);
  auto row_of = [&](int64_t r) -> int64_t {
    return a.route_row ? (int64_t)a.route_row[r] : a.sel[r] * a.T + t;
  };
  if (a.vec) {
    for (int64_t d0 = (int64_t)threadIdx.x * V; d0 < a.D; d0 += 256 * V) {
      float acc[V];
#pragma unroll
      for (int e = 0; e < V; ++e) acc[e] = 0.f;
      if (ok) {
        for (int64_t s0 = 0; s0 < a.k; s0 += G) {
          u32x4_t v[G];
          float w[G];
#pragma unroll
          for (int u = 0; u < G; ++u) {
            if (s0 + u < a.k) {
              const int64_t r = t * a.k + s0 + u;
              w[u] = s0 == 0 ? w0[u] : load_weight<T>(a.w, a.w_dtype, r);
              const int64_t row = s0 == 0 ? row0[u] : row_of(r);
              v[u] = *reinterpret_cast<const u32x4_t*>(ybase + row * a.D + d0);
            }
          }
#pragma unroll
          for (int u = 0; u < G; ++u) {
            if (s0 + u < a.k) {
#pragma unroll
              for (int e = 0; e < V; ++e) {
                const float x = Num<T>::round(chunk_elem<T>(v[u], e) * w[u]);
                acc[e] = (s0 + u == 0) ? x : Num<T>::round(acc[e] + x);
              }
            }
          }
        }
      }
      u32x4_t o = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < V; ++e) chunk_put<T>(o, e, acc[e]);
      *reinterpret_cast<u32x4_t*>(out + d0) = o;
    }
    return;
  }
  for (int64_t d0 = (int64_t)threadIdx.x * 4; d0 < a.D; d0 += 256 * 4) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    if (ok) {
      for (int64_t s = 0; s < a.k; ++s) {
        const int64_t r = t * a.k + s;
        const float w = load_weight<T>(a.w, a.w_dtype, r);
        const T* y = ybase + row_of(r) * a.D;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (d0 + c < a.D) {
            const float v = Num<T>::round(Num<T>::load(y + d0 + c) * w);
            acc[c] = (s == 0) ? v : Num<T>::round(acc[c] + v);
          }
        }
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (d0 + c < a.D) Num<T>::store(out + d0 + c, acc[c]);
  }
}

// ------------------------------------------------------------------ route packing ----
// Route r = t*k + s belongs to bucket sel[r] (an expert) or, for an index outside [0, E), to
// bucket E (never computed).  The routes are cut into chunks of 256 consecutive routes, one
// workgroup each:
//   rank kernel  rank[r]      = routes r' < r of r's chunk in r's bucket,
//                counts[b][c] = routes of chunk c in bucket b (bucket-major);
//   plan kernel  counts[b][c] -> routes of chunks before c in bucket b (in place; one
//                wavefront scans a bucket's chunk counts 64 at a time),
//                off[e]       = first packed row of expert e (experts in index order),
//                grp1 / grp2  = m-tile tables of the two grouped GEMMs (with tail1 / tail2 > 0
//                               an expert's last m-tile of fewer rows goes to grp1t / grp2t,
//                               the tables of the tail launches);
//   route rows   row(r) = off[e] + counts[e][c] + rank[r]; row_token[row(r)] = t, the x row the
//                gate/up GEMM reads for packed row row(r).
// Packed rows of an expert are therefore its routes in increasing r.
constexpr int kRankWaves = 4;
constexpr int kMaxSparseExperts = 2048;
constexpr int kPlanThreads = 1024;

struct PackArgs {
  const int64_t* sel;
  int32_t* rank;
  int32_t* counts;     // [E + 1][S]
  int32_t* off;        // [E + 1]
  int32_t* grp1;       // m-tiles of bm1 rows
  int32_t* grp2;       // m-tiles of bm2 rows
  int32_t* grp1t;      // tail m-tiles of the gate/up GEMM (tail1 > 0; plan kernel only)
  int32_t* grp2t;      // tail m-tiles of the down GEMM (tail2 > 0; plan kernel only)
  int32_t* route_row;  // [R], -1 for bucket E
  int32_t* row_token;  // [R] token of each packed row
  int64_t R, k, E, S, chunk;
  int32_t bm1, bm2;
  int32_t tail1, tail2;  // rows below which an expert's last m-tile is a tail (0: none)
};

static int64_t route_chunk(int64_t) { return 64 * kRankWaves; }

// Workgroup barrier for data passed through LDS only: waits for this wavefront's LDS accesses,
// not for its global stores (which a __syncthreads() waits for, and which no later step of
// these kernels reads back).  The empty assembly statements keep the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void lds_sync() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0), vmcnt unchanged
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// One workgroup per chunk of 256 routes, one wavefront per 64 of them: the lanes holding the
// same bucket find each other through one ballot per bucket-index bit; a route's rank is the
// count of such lanes below it plus the bucket's routes in the chunk's earlier wavefronts, and
// the chunk's count of a bucket sums its four wavefronts' counts.
__global__ __launch_bounds__(256) void moe_rank_kernel(PackArgs a) {
  extern __shared__ int32_t hist[];  // [kRankWaves][E + 1]
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int64_t E1 = a.E + 1;
  const int64_t c = blockIdx.x;
  int32_t* h = hist + w * E1;
  for (int64_t b = lane; b < E1; b += 64) h[b] = 0;
  const int64_t r = c * (64 * kRankWaves) + tid;
  const bool valid = r < a.R;
  int b = (int)a.E;
  if (valid) {
    const int64_t e = a.sel[r];
    if (e >= 0 && e < a.E) b = (int)e;
  }
  const int nbits = 32 - __clz((int)a.E);
  uint64_t same = __ballot(valid);
  for (int bit = 0; bit < nbits; ++bit) {
    const bool on = (b >> bit) & 1;
    const uint64_t m = __ballot(valid && on);
    same &= on ? m : ~m;
  }
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int lower = __popcll(same & below);
  if (valid && lower == 0) h[b] = __popcll(same);
  lds_sync();
  if (valid) {
    int32_t before = 0;
    for (int v = 0; v < w; ++v) before += hist[v * E1 + b];
    a.rank[r] = before + lower;
  }
  for (int64_t q = tid; q < E1; q += 64 * kRankWaves) {
    int32_t n = 0;
#pragma unroll
    for (int v = 0; v < kRankWaves; ++v) n += hist[v * E1 + q];
    a.counts[q * a.S + c] = n;
  }
}

// Inclusive prefix sum over the 64 lanes of a wavefront.
__device__ __forceinline__ int32_t wave_incl_scan(int32_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int32_t o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

// One workgroup.  First, wavefront w scans the chunk counts of buckets w, w + 16, ... (64 chunks
// at a time, eight loads in flight) into routes of earlier chunks and records each bucket's
// size.  Then thread i owns buckets [i*per, (i+1)*per), and a workgroup scan over the threads
// of (rows, main and tail m-tiles of both GEMMs) places each expert's rows and m-tiles.
__global__ __launch_bounds__(kPlanThreads) void moe_plan_kernel(PackArgs a) {
  constexpr int W = kPlanThreads / 64;
  __shared__ int32_t size_l[kMaxSparseExperts + 1];
  __shared__ int32_t wsum[W][5];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int64_t E = a.E, E1 = E + 1;
  // Up to 512 chunks (131072 routes): the loads of NBK buckets of a wavefront go out together
  // (the counts were just written by every XCD, so each load waits for memory).
  constexpr int NBK = 8;
  if (a.S <= 64 * 8) {
    for (int64_t bb = w; bb < E1; bb += (int64_t)W * NBK) {
      int32_t v[NBK][8];
#pragma unroll
      for (int j = 0; j < NBK; ++j) {
        const int64_t b = bb + (int64_t)W * j;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int64_t c = 64 * u + lane;
          v[j][u] = (b < E1 && c < a.S) ? a.counts[b * a.S + c] : 0;
        }
      }
#pragma unroll
      for (int j = 0; j < NBK; ++j) {
        const int64_t b = bb + (int64_t)W * j;
        if (b >= E1) break;
        int32_t carry = 0;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (64 * u >= a.S) break;
          const int32_t inc = wave_incl_scan(v[j][u]);
          const int64_t c = 64 * u + lane;
          if (c < a.S) a.counts[b * a.S + c] = carry + inc - v[j][u];
          carry += __shfl(inc, 63, 64);
        }
        if (lane == 0) size_l[b] = carry;
      }
    }
  } else {
    for (int64_t b = w; b < E1; b += W) {
      int32_t carry = 0;
      for (int64_t c0 = 0; c0 < a.S; c0 += 64 * 8) {
        int32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int64_t c = c0 + 64 * u + lane;
          v[u] = c < a.S ? a.counts[b * a.S + c] : 0;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int32_t inc = wave_incl_scan(v[u]);
          const int64_t c = c0 + 64 * u + lane;
          if (c < a.S) a.counts[b * a.S + c] = carry + inc - v[u];
          carry += __shfl(inc, 63, 64);
        }
      }
      if (lane == 0) size_l[b] = carry;
    }
  }
  lds_sync();
  const int64_t per = (E1 + kPlanThreads - 1) / kPlanThreads;
  const int64_t b0 = std::min(E1, tid * per), b1 = std::min(E1, b0 + per);
  // m-tiles of an expert of n rows in a table of bm-row tiles: main ones, and whether the last
  // one (fewer than `tail` rows) is a tail
  auto tiles = [](int32_t n, int32_t bm, int32_t tail, int32_t& main, int32_t& tl) {
    const int32_t all = (n + bm - 1) / bm;
    tl = (all > 0 && n - (all - 1) * bm < tail) ? 1 : 0;
    main = all - tl;
  };
  // per thread: rows, gate/up main and tail m-tiles, down main and tail m-tiles
  int32_t q[5] = {0, 0, 0, 0, 0};
  for (int64_t b = b0; b < b1; ++b) {
    if (b < E) {
      const int32_t n = size_l[b];
      int32_t m1, x1, m2, x2;
      tiles(n, a.bm1, a.tail1, m1, x1);
      tiles(n, a.bm2, a.tail2, m2, x2);
      q[0] += n; q[1] += m1; q[2] += x1; q[3] += m2; q[4] += x2;
    }
  }
  // exclusive scan over the threads: wavefront scans, then the sums of earlier wavefronts
  int32_t inc[5], pre[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    inc[i] = wave_incl_scan(q[i]);
    if (lane == 63) wsum[w][i] = inc[i];
  }
  lds_sync();
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    pre[i] = 0;
    for (int v = 0; v < w; ++v) pre[i] += wsum[v][i];
  }
  int32_t row0 = pre[0] + inc[0] - q[0];
  int32_t j1 = pre[1] + inc[1] - q[1], k1 = pre[2] + inc[2] - q[2];
  int32_t j2 = pre[3] + inc[3] - q[3], k2 = pre[4] + inc[4] - q[4];
  auto put = [](int32_t* table, int32_t j, int32_t e, int32_t first, int32_t end) {
    int32_t* g = table + kGrpHeader + kGrpStride * j;
    g[0] = e; g[1] = first; g[2] = end; g[3] = 0;
  };
  for (int64_t b = b0; b < b1; ++b) {
    const int32_t n = size_l[b];
    a.off[b] = row0;
    if (b < E) {
      int32_t m1, x1, m2, x2;
      tiles(n, a.bm1, a.tail1, m1, x1);
      tiles(n, a.bm2, a.tail2, m2, x2);
      for (int32_t t = 0; t < m1; ++t) put(a.grp1, j1++, (int32_t)b, row0 + t * a.bm1, row0 + n);
      if (x1) put(a.grp1t, k1++, (int32_t)b, row0 + m1 * a.bm1, row0 + n);
      for (int32_t t = 0; t < m2; ++t) put(a.grp2, j2++, (int32_t)b, row0 + t * a.bm2, row0 + n);
      if (x2) put(a.grp2t, k2++, (int32_t)b, row0 + m2 * a.bm2, row0 + n);
      row0 += n;
    }
  }
  if (tid == kPlanThreads - 1) {
    a.grp1[0] = pre[1] + inc[1];
    a.grp2[0] = pre[3] + inc[3];
    if (a.tail1 > 0) a.grp1t[0] = pre[2] + inc[2];
    if (a.tail2 > 0) a.grp2t[0] = pre[4] + inc[4];
  }
}

// Packed row of every route (route_row[r], -1 for an invalid expert index) and the token of
// every packed row (row_token[row] = r / k): the gate/up GEMM reads its A rows through that
// table, so no copy of x is made.  One thread per route.
__global__ __launch_bounds__(256) void moe_route_rows_kernel(PackArgs a) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= a.R) return;
  const int64_t e = a.sel[r];
  const bool ok = e >= 0 && e < a.E;
  int64_t row = -1;
  if (ok) row = (int64_t)a.off[e] + a.counts[e * a.S + r / a.chunk] + a.rank[r];
  a.route_row[r] = (int32_t)row;
  if (ok) a.row_token[row] = (int32_t)(r / a.k);
}

// Route packing of a small call in one workgroup: the rank, plan and route-row kernels above
// in one launch, with the same route rows, token table, expert offsets and m-tile tables
// (a few-token call otherwise spends three kernel latencies on eight routes).  Thread r owns
// route r; the lanes of one wavefront holding the same bucket find each other by ballots, and
// bucket b's count per wavefront goes to LDS; thread b then turns the 16 counts into the routes
// of earlier wavefronts, and a workgroup scan over the buckets places rows and m-tiles.
// The workgroup has the fewest of 2 / 4 / 8 / 16 wavefronts that give every route and every
// bucket a thread.  Calls of up to 4096 routes over at most 127 experts take the same kernel
// with 16 wavefronts and up to four passes over the routes: pass p gives thread t route
// 1024 p + t, and the per-wavefront counts of every pass are prefixed in route order.
constexpr int kSmallPackRoutes = 1024;  // routes per pass (one per thread)
constexpr int kSmallPackBuckets = 512;  // experts + 1 (the bucket of invalid indices)
constexpr int kMultiPackPasses = 4;     // passes of the multi-pass form
constexpr int kMultiPackBuckets = 128;  // its experts + 1

template <int WAVES, int PASSES = 1, int BUCKETS = kSmallPackBuckets>
__global__ __launch_bounds__(WAVES * 64) void moe_pack_small_kernel(PackArgs a) {
  constexpr int NT = WAVES * 64;
  static_assert(NT <= kSmallPackRoutes, "one thread per route of a pass");
  static_assert(PASSES == 1 || BUCKETS <= NT, "one thread per bucket (the launcher checks it otherwise)");
  // row v = p * WAVES + w: counts of wavefront w in pass p (route order)
  __shared__ int32_t cnt[PASSES * WAVES][BUCKETS];
  __shared__ int32_t first_row[BUCKETS];
  __shared__ int32_t wsum[WAVES][3];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int E = (int)a.E, E1 = E + 1;
  // each wavefront zeroes and writes only its own rows of cnt
#pragma unroll
  for (int p = 0; p < PASSES; ++p)
    for (int b = lane; b < E1; b += 64) cnt[p * WAVES + w][b] = 0;
  const int nbits = 32 - __clz(E);
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  bool valid[PASSES];
  int bucket[PASSES], lower[PASSES];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int64_t r = (int64_t)p * NT + tid;
    valid[p] = r < a.R;
    bucket[p] = E;
    if (valid[p]) {
      const int64_t e = a.sel[r];
      if (e >= 0 && e < a.E) bucket[p] = (int)e;
    }
    uint64_t same = __ballot(valid[p]);
    for (int bit = 0; bit < nbits; ++bit) {
      const bool on = (bucket[p] >> bit) & 1;
      const uint64_t m = __ballot(valid[p] && on);
      same &= on ? m : ~m;
    }
    lower[p] = __popcll(same & below);
    if (valid[p] && lower[p] == 0) cnt[p * WAVES + w][bucket[p]] = __popcll(same);
  }
  lds_sync();
  int32_t n = 0;  // routes of bucket tid
  if (tid < E1) {
    for (int v = 0; v < PASSES * WAVES; ++v) {
      const int32_t c = cnt[v][tid];
      cnt[v][tid] = n;
      n += c;
    }
  }
  const bool expert = tid < E;
  const int32_t rows = expert ? n : 0;
  const int32_t t1 = expert ? (n + a.bm1 - 1) / a.bm1 : 0;
  const int32_t t2 = expert ? (n + a.bm2 - 1) / a.bm2 : 0;
  const int32_t ir = wave_incl_scan(rows), i1 = wave_incl_scan(t1), i2 = wave_incl_scan(t2);
  if (lane == 63) {
    wsum[w][0] = ir;
    wsum[w][1] = i1;
    wsum[w][2] = i2;
  }
  lds_sync();
  int32_t pr = 0, p1 = 0, p2 = 0;
  for (int v = 0; v < w; ++v) {
    pr += wsum[v][0];
    p1 += wsum[v][1];
    p2 += wsum[v][2];
  }
  const int32_t row0 = pr + ir - rows;
  if (tid < E1) {
    first_row[tid] = row0;
    a.off[tid] = row0;
  }
  if (expert) {
    int32_t j = p1 + i1 - t1;
    for (int32_t m = 0; m < n; m += a.bm1, ++j) {
      int32_t* g = a.grp1 + kGrpHeader + kGrpStride * j;
      g[0] = tid; g[1] = row0 + m; g[2] = row0 + n; g[3] = 0;
    }
    j = p2 + i2 - t2;
    for (int32_t m = 0; m < n; m += a.bm2, ++j) {
      int32_t* g = a.grp2 + kGrpHeader + kGrpStride * j;
      g[0] = tid; g[1] = row0 + m; g[2] = row0 + n; g[3] = 0;
    }
  }
  if (tid == WAVES * 64 - 1) {
    a.grp1[0] = p1 + i1;
    a.grp2[0] = p2 + i2;
  }
  lds_sync();
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    if (valid[p]) {
      const int64_t r = (int64_t)p * NT + tid;
      int32_t row = -1;
      if (bucket[p] < E) {
        row = first_row[bucket[p]] + cnt[p * WAVES + w][bucket[p]] + lower[p];
        a.row_token[row] = (int32_t)(r / a.k);
      }
      a.route_row[r] = row;
    }
  }
}

// Workspace of the sparse path (byte offsets, 256-byte aligned).
struct SparseLayout {
  int64_t y, act, rank, route, token, counts, off, grp1, grp2, grp1t, grp2t, total;
};

static SparseLayout sparse_layout(int elt, int64_t R, int64_t E, int64_t D, int64_t I) {
  auto al = [](int64_t b) { return (b + 255) & ~int64_t(255); };
  const int64_t S = cdiv(R, route_chunk(R));
  // Tile tables sized for the smallest m-tile height of the grouped entries.
  const int64_t tiles = cdiv(R, kMinGroupedTileRows) + std::min(E, R);
  SparseLayout L;
  int64_t p = 0;
  L.y = p; p += al(R * D * elt);  // packed down-projection rows
  L.act = p; p += al(R * I * elt);
  L.rank = p; p += al(R * 4);
  L.route = p; p += al(R * 4);
  L.token = p; p += al(R * 4);
  L.counts = p; p += al(S * (E + 1) * 4);
  L.off = p; p += al((E + 1) * 4);
  L.grp1 = p; p += al((kGrpHeader + kGrpStride * tiles) * 4);
  L.grp2 = p; p += al((kGrpHeader + kGrpStride * tiles) * 4);
  // tail tables: at most one m-tile per expert
  L.grp1t = p; p += al((kGrpHeader + kGrpStride * std::min(E, R)) * 4);
  L.grp2t = p; p += al((kGrpHeader + kGrpStride * std::min(E, R)) * 4);
  L.total = p;
  return L;
}

static int launch_combine(int dtype, CombineArgs c, hipStream_t s) {
  if (c.T > 0x7fffffffLL) return fail(BIOPS_ERR_ARG, "too many tokens");
  const int elt = dtype_bytes(dtype);
  c.vec = (c.D * elt) % 16 == 0 && reinterpret_cast<uintptr_t>(c.y) % 16 == 0 &&
          reinterpret_cast<uintptr_t>(c.out) % 16 == 0;
  switch (dtype) {
    case BIOPS_F32: hipLaunchKernelGGL(moe_combine_kernel<float>, dim3((unsigned)c.T), dim3(256), 0, s, c); break;
    case BIOPS_F16: hipLaunchKernelGGL(moe_combine_kernel<f16_t>, dim3((unsigned)c.T), dim3(256), 0, s, c); break;
    default: hipLaunchKernelGGL(moe_combine_kernel<bf16_t>, dim3((unsigned)c.T), dim3(256), 0, s, c); break;
  }
  return check_launch("moe_combine_kernel");
}

// Shared argument checks and the two expert GEMMs' operand layouts.
struct ExpertGemms {
  BmmArgs gu, dn;
  bool gu_kmajor, dn_kmajor;
};

static int expert_gemms(int64_t tokens, int64_t experts, int64_t hidden, int64_t inter, const void* x,
                        int64_t sx, const void* gate, int64_t sgE, int64_t sgI, int64_t sgD, const void* up,
                        int64_t suE, int64_t suI, int64_t suD, const void* down, int64_t sdE, int64_t sdD,
                        int64_t sdI, ExpertGemms& g) {
  if (sgE != suE || sgI != suI || sgD != suD)
    return fail(BIOPS_ERR_LAYOUT, "gate and up weights must share strides");
  int64_t ldb;
  // act[., i]: B = gate_e / up_e viewed as [I, D] (column i, K = d).
  if (!b_layout(hidden, inter, sgD, sgI, g.gu_kmajor, ldb))
    return fail(BIOPS_ERR_LAYOUT, "gate/up weights need a unit stride");
  g.gu = BmmArgs{};
  g.gu.A = x; g.gu.B = gate; g.gu.B2 = up;
  g.gu.M = tokens; g.gu.N = inter; g.gu.K = hidden;
  g.gu.lda = sx; g.gu.ldb = ldb;
  g.gu.nb1 = experts; g.gu.nb2 = 1; g.gu.gB = 1;
  g.gu.sB1 = sgE;
  // y[., d] = act[., :] . down_e[d, :]
  if (!b_layout(inter, hidden, sdI, sdD, g.dn_kmajor, ldb))
    return fail(BIOPS_ERR_LAYOUT, "down weights need a unit stride");
  g.dn = BmmArgs{};
  g.dn.B = down;
  g.dn.M = tokens; g.dn.N = hidden; g.dn.K = inter;
  g.dn.lda = inter; g.dn.ldb = ldb; g.dn.ldc = hidden;
  g.dn.nb1 = experts; g.dn.nb2 = 1; g.dn.gB = 1;
  g.dn.sB1 = sdE;
  return BIOPS_OK;
}

}  // namespace biops

using namespace biops;

extern "C" int64_t biops_moe_workspace_size(int dtype, int64_t tokens, int64_t experts,
                                            int64_t hidden, int64_t inter) {
  const int elt = dtype_bytes(dtype);
  if (elt == 0 || tokens < 0 || experts < 0 || hidden < 0 || inter < 0) return -1;
  const int64_t act = experts * tokens * inter;
  const int64_t act_pad = (act + 63) & ~int64_t(63);
  return (act_pad + experts * tokens * hidden) * elt;
}

extern "C" int biops_moe(int dtype, int64_t tokens, int64_t experts, int64_t hidden, int64_t inter,
                         int64_t top_k, const void* x, int64_t sx, const void* gate, int64_t sgE,
                         int64_t sgI, int64_t sgD, const void* up, int64_t suE, int64_t suI,
                         int64_t suD, const void* down, int64_t sdE, int64_t sdD, int64_t sdI,
                         const void* weights, int w_dtype, const int64_t* sel, void* out,
                         int32_t* bad_index, void* workspace, int64_t workspace_bytes,
                         void* stream) {
  if (!is_float_dtype(dtype) || !is_float_dtype(w_dtype))
    return fail(BIOPS_ERR_DTYPE, "unsupported MoE dtype");
  if (tokens < 0 || experts <= 0 || hidden < 0 || inter < 0 || top_k < 0)
    return fail(BIOPS_ERR_ARG, "invalid MoE sizes");
  if (tokens == 0 || hidden == 0) return BIOPS_OK;
  ExpertGemms g;
  int rc = expert_gemms(tokens, experts, hidden, inter, x, sx, gate, sgE, sgI, sgD, up, suE, suI, suD, down,
                        sdE, sdD, sdI, g);
  if (rc != BIOPS_OK) return rc;
  const int64_t need = biops_moe_workspace_size(dtype, tokens, experts, hidden, inter);
  if (workspace_bytes < need) return fail(BIOPS_ERR_SIZE, "workspace %lld < %lld bytes",
                                          (long long)workspace_bytes, (long long)need);
  const int elt = dtype_bytes(dtype);
  hipStream_t s = (hipStream_t)stream;
  char* ws = reinterpret_cast<char*>(workspace);
  const int64_t act_elems = (experts * tokens * inter + 63) & ~int64_t(63);
  void* act = ws;
  void* y = ws + act_elems * elt;

  if (top_k > 0) {
    // act[e, t, i] and y[e, t, d] for every expert: A broadcast over the experts.
    g.gu.C = act; g.gu.ldc = inter; g.gu.sA1 = 0; g.gu.sC1 = tokens * inter;
    if ((rc = launch_bmm(dtype, g.gu, kEpiSwiglu, g.gu_kmajor, s)) != BIOPS_OK) return rc;
    g.dn.A = act; g.dn.C = y; g.dn.sA1 = tokens * inter; g.dn.sC1 = tokens * hidden;
    if ((rc = launch_bmm(dtype, g.dn, kEpiPlain, g.dn_kmajor, s)) != BIOPS_OK) return rc;
  }
  CombineArgs c{y, weights, sel, nullptr, out, bad_index, tokens, hidden, experts, top_k, w_dtype, 0};
  return launch_combine(dtype, c, s);
}

extern "C" int64_t biops_moe_sparse_workspace_size(int dtype, int64_t tokens, int64_t top_k,
                                                   int64_t experts, int64_t hidden, int64_t inter) {
  const int elt = dtype_bytes(dtype);
  if (elt == 0 || tokens < 0 || top_k < 0 || experts <= 0 || hidden < 0 || inter < 0) return -1;
  if (experts > kMaxSparseExperts) return -1;
  return sparse_layout(elt, tokens * top_k, experts, hidden, inter).total;
}

namespace biops {

// Size checks shared by the two sparse entry points (BIOPS_OK, or the failure code with the
// message set).  Pure host arithmetic: no HIP call.
static int sparse_sizes_ok(int dtype, int w_dtype, int64_t tokens, int64_t experts, int64_t hidden,
                           int64_t inter, int64_t top_k) {
  if (!is_float_dtype(dtype) || !is_float_dtype(w_dtype))
    return fail(BIOPS_ERR_DTYPE, "unsupported MoE dtype");
  if (tokens < 0 || experts <= 0 || hidden < 0 || inter < 0 || top_k < 0)
    return fail(BIOPS_ERR_ARG, "invalid MoE sizes");
  if (experts > kMaxSparseExperts)
    return fail(BIOPS_ERR_ARG, "sparse MoE supports up to %d experts", kMaxSparseExperts);
  if (tokens * top_k >= (int64_t(1) << 31)) return fail(BIOPS_ERR_SIZE, "too many routes");
  return BIOPS_OK;
}

// The sparse evaluation on a caller-provided workspace (sizes already checked).  Every route
// table and packed matrix in the workspace is written before it is read within the call, so
// the workspace needs no clearing and keeps nothing from one call to the next.
static int moe_sparse_run(int dtype, int64_t tokens, int64_t experts, int64_t hidden, int64_t inter,
                          int64_t top_k, const void* x, int64_t sx, const void* gate, int64_t sgE,
                          int64_t sgI, int64_t sgD, const void* up, int64_t suE, int64_t suI,
                          int64_t suD, const void* down, int64_t sdE, int64_t sdD, int64_t sdI,
                          const void* weights, int w_dtype, const int64_t* sel, void* out,
                          int32_t* bad_index, void* workspace, int64_t workspace_bytes,
                          void* stream) {
  if (tokens == 0 || hidden == 0) return BIOPS_OK;
  const int64_t R = tokens * top_k;
  ExpertGemms g;
  int rc = expert_gemms(tokens, experts, hidden, inter, x, sx, gate, sgE, sgI, sgD, up, suE, suI, suD, down,
                        sdE, sdD, sdI, g);
  if (rc != BIOPS_OK) return rc;
  const int elt = dtype_bytes(dtype);
  const SparseLayout L = sparse_layout(elt, R, experts, hidden, inter);
  if (workspace_bytes < L.total) return fail(BIOPS_ERR_SIZE, "workspace %lld < %lld bytes",
                                             (long long)workspace_bytes, (long long)L.total);
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
    return fail(BIOPS_ERR_LAYOUT, "workspace must be 256-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  char* ws = reinterpret_cast<char*>(workspace);
  int32_t* route_row = reinterpret_cast<int32_t*>(ws + L.route);

  if (R > 0) {
    // Grouped GEMM operands: packed rows, one row group per expert; the gate/up GEMM reads the
    // x row of each packed row through the row -> token table.
    int32_t* row_token = reinterpret_cast<int32_t*>(ws + L.token);
    g.gu.a_rows = row_token;
    g.gu.C = ws + L.act; g.gu.ldc = inter;
    g.gu.grp = reinterpret_cast<const int32_t*>(ws + L.grp1);
    g.dn.A = ws + L.act;
    g.dn.C = ws + L.y;
    g.dn.grp = reinterpret_cast<const int32_t*>(ws + L.grp2);
    for (BmmArgs* b : {&g.gu, &g.dn}) {
      b->grp_rows = R;
      b->grp_groups = experts;
      b->M = cdiv(R, experts);  // mean rows per expert, for the tile choice
    }
    const int bm1 = grouped_tile_rows(dtype, g.gu, kEpiSwiglu, g.gu_kmajor);
    const int bm2 = grouped_tile_rows(dtype, g.dn, kEpiPlain, g.dn_kmajor);
    if (bm1 < kMinGroupedTileRows || bm2 < kMinGroupedTileRows) return fail(BIOPS_ERR_ARG, "no grouped GEMM tile");

    PackArgs p{};
    p.sel = sel;
    p.rank = reinterpret_cast<int32_t*>(ws + L.rank);
    p.counts = reinterpret_cast<int32_t*>(ws + L.counts);
    p.off = reinterpret_cast<int32_t*>(ws + L.off);
    p.grp1 = reinterpret_cast<int32_t*>(ws + L.grp1);
    p.grp2 = reinterpret_cast<int32_t*>(ws + L.grp2);
    p.route_row = route_row;
    p.row_token = row_token;
    p.R = R; p.k = top_k; p.E = experts;
    p.chunk = route_chunk(R);
    p.S = cdiv(R, p.chunk);
    p.bm1 = bm1; p.bm2 = bm2;
    p.grp1t = reinterpret_cast<int32_t*>(ws + L.grp1t);
    p.grp2t = reinterpret_cast<int32_t*>(ws + L.grp2t);
    const bool small = R <= kSmallPackRoutes && experts + 1 <= kSmallPackBuckets;
    // Tail m-tiles go to separate launches on the weight-streaming tile (plan kernel path).
    p.tail1 = small ? 0 : grouped_tail_rows(dtype, g.gu, kEpiSwiglu, g.gu_kmajor);
    p.tail2 = small ? 0 : grouped_tail_rows(dtype, g.dn, kEpiPlain, g.dn_kmajor);
    // up to 4096 routes over at most 127 experts without tails: the multi-pass one-workgroup
    // packing (C5 at 256 tokens: one kernel of about 5 us against the three of the plan path)
    const bool multi = !small && R <= (int64_t)kMultiPackPasses * kSmallPackRoutes &&
                       experts + 1 <= kMultiPackBuckets && p.tail1 == 0 && p.tail2 == 0;
    if (small) {
      const int64_t threads = std::max<int64_t>(R, experts + 1);
      if (threads <= 128) hipLaunchKernelGGL(moe_pack_small_kernel<2>, dim3(1), dim3(128), 0, s, p);
      else if (threads <= 256) hipLaunchKernelGGL(moe_pack_small_kernel<4>, dim3(1), dim3(256), 0, s, p);
      else if (threads <= 512) hipLaunchKernelGGL(moe_pack_small_kernel<8>, dim3(1), dim3(512), 0, s, p);
      else hipLaunchKernelGGL(moe_pack_small_kernel<16>, dim3(1), dim3(1024), 0, s, p);
      if ((rc = check_launch("moe_pack_small_kernel")) != BIOPS_OK) return rc;
    } else if (multi) {
      if (R <= 2 * kSmallPackRoutes)
        hipLaunchKernelGGL((moe_pack_small_kernel<16, 2, kMultiPackBuckets>), dim3(1), dim3(1024), 0, s, p);
      else
        hipLaunchKernelGGL((moe_pack_small_kernel<16, kMultiPackPasses, kMultiPackBuckets>), dim3(1), dim3(1024), 0,
                           s, p);
      if ((rc = check_launch("moe_pack_small_kernel")) != BIOPS_OK) return rc;
    } else {
      const size_t hist_bytes = (size_t)kRankWaves * (experts + 1) * sizeof(int32_t);
      hipLaunchKernelGGL(moe_rank_kernel, dim3((unsigned)p.S), dim3(64 * kRankWaves), hist_bytes, s, p);
      if ((rc = check_launch("moe_rank_kernel")) != BIOPS_OK) return rc;
      hipLaunchKernelGGL(moe_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, p);
      if ((rc = check_launch("moe_plan_kernel")) != BIOPS_OK) return rc;
      hipLaunchKernelGGL(moe_route_rows_kernel, dim3((unsigned)cdiv(R, 256)), dim3(256), 0, s, p);
      if ((rc = check_launch("moe_route_rows_kernel")) != BIOPS_OK) return rc;
    }
    // the tail launches: at most one m-tile per expert
    auto tail_of = [&](BmmArgs t, int32_t* table) {
      t.grp = table;
      t.grp_rows = t.grp_groups = std::min<int64_t>(R, experts);
      return t;
    };
    if ((rc = launch_bmm(dtype, g.gu, kEpiSwiglu, g.gu_kmajor, s)) != BIOPS_OK) return rc;
    if (p.tail1 > 0 && (rc = launch_grouped_tail(dtype, tail_of(g.gu, p.grp1t), kEpiSwiglu, s)) != BIOPS_OK)
      return rc;
    if ((rc = launch_bmm(dtype, g.dn, kEpiPlain, g.dn_kmajor, s)) != BIOPS_OK) return rc;
    if (p.tail2 > 0 && (rc = launch_grouped_tail(dtype, tail_of(g.dn, p.grp2t), kEpiPlain, s)) != BIOPS_OK)
      return rc;
  }
  CombineArgs c{ws + L.y, weights, sel, route_row, out, bad_index, tokens, hidden, experts, top_k, w_dtype, 0};
  return launch_combine(dtype, c, s);
}

// Scratch of biops_moe_sparse_noalloc: a library-owned device array, one copy on every GPU the
// library runs on, held until the process ends.  On the host the name `scratch` is only a
// stand-in for the device symbol; its device address on each GPU comes from
// hipGetSymbolAddress (noalloc_scratch below) and only that address reaches the kernels.
static __device__ __align__(256) char scratch[BIOPS_MOE_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxScratchDevices];
std::mutex g_scratch_mutex;

// Order of the calls that share a device's array: each call's stream waits (on the device, not
// the host) for an event recorded after the previous call's last kernel, whatever stream that
// call used.  The mutex orders the host side: the wait, the launches and the record of one
// call are not interleaved with another thread's.
struct ScratchOrder {
  std::mutex m;
  hipEvent_t done = nullptr;  // created on the device's first call
  bool recorded = false;
};
ScratchOrder g_scratch_order[kMaxScratchDevices];
}  // namespace

// Device address of `scratch` on the current device, looked up once per device (with that
// device current) and cached.
static int noalloc_scratch(void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return fail(BIOPS_ERR_HIP, "no current HIP device (or device index >= %d)", kMaxScratchDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr)
        return fail(BIOPS_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  return BIOPS_OK;
}

}  // namespace biops

extern "C" int biops_moe_sparse(int dtype, int64_t tokens, int64_t experts, int64_t hidden,
                                int64_t inter, int64_t top_k, const void* x, int64_t sx,
                                const void* gate, int64_t sgE, int64_t sgI, int64_t sgD,
                                const void* up, int64_t suE, int64_t suI, int64_t suD,
                                const void* down, int64_t sdE, int64_t sdD, int64_t sdI,
                                const void* weights, int w_dtype, const int64_t* sel, void* out,
                                int32_t* bad_index, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  const int rc = sparse_sizes_ok(dtype, w_dtype, tokens, experts, hidden, inter, top_k);
  if (rc != BIOPS_OK) return rc;
  return moe_sparse_run(dtype, tokens, experts, hidden, inter, top_k, x, sx, gate, sgE, sgI, sgD, up, suE,
                        suI, suD, down, sdE, sdD, sdI, weights, w_dtype, sel, out, bad_index, workspace,
                        workspace_bytes, stream);
}

extern "C" int biops_moe_sparse_noalloc(int dtype, int64_t tokens, int64_t experts, int64_t hidden,
                                        int64_t inter, int64_t top_k, const void* x, int64_t sx,
                                        const void* gate, int64_t sgE, int64_t sgI, int64_t sgD,
                                        const void* up, int64_t suE, int64_t suI, int64_t suD,
                                        const void* down, int64_t sdE, int64_t sdD, int64_t sdI,
                                        const void* weights, int w_dtype, const int64_t* sel, void* out,
                                        int32_t* bad_index, void* stream) {
  int rc = sparse_sizes_ok(dtype, w_dtype, tokens, experts, hidden, inter, top_k);
  if (rc != BIOPS_OK) return rc;
  const int64_t need = sparse_layout(dtype_bytes(dtype), tokens * top_k, experts, hidden, inter).total;
  if (need > BIOPS_MOE_NOALLOC_SCRATCH_BYTES)
    return fail(BIOPS_ERR_SIZE,
                "biops_moe_sparse_noalloc: %lld tokens x top-%lld need %lld bytes of scratch, more than the "
                "%lld-byte static array; use biops_moe_sparse with a workspace",
                (long long)tokens, (long long)top_k, (long long)need,
                (long long)BIOPS_MOE_NOALLOC_SCRATCH_BYTES);
  if (tokens == 0 || hidden == 0) return BIOPS_OK;
  void* ws = nullptr;
  if ((rc = noalloc_scratch(&ws)) != BIOPS_OK) return rc;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(BIOPS_ERR_HIP, "no current HIP device");
  hipStream_t s = (hipStream_t)stream;
  // Under stream capture the wait and the record are left out: a captured stream cannot wait on
  // an event recorded outside the capture, and a graph's replays on one stream run in order.
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &capture) != hipSuccess)
    return fail(BIOPS_ERR_HIP, "hipStreamIsCapturing failed");
  const bool order = capture == hipStreamCaptureStatusNone;
  ScratchOrder& o = g_scratch_order[dev];
  std::lock_guard<std::mutex> lock(o.m);
  if (order) {
    if (o.done == nullptr) {
      const hipError_t e = hipEventCreateWithFlags(&o.done, hipEventDisableTiming);
      if (e != hipSuccess) return fail(BIOPS_ERR_HIP, "hipEventCreateWithFlags: %s", hipGetErrorString(e));
    }
    if (o.recorded) {
      const hipError_t e = hipStreamWaitEvent(s, o.done, 0);
      if (e != hipSuccess) return fail(BIOPS_ERR_HIP, "hipStreamWaitEvent: %s", hipGetErrorString(e));
    }
  }
  rc = moe_sparse_run(dtype, tokens, experts, hidden, inter, top_k, x, sx, gate, sgE, sgI, sgD, up, suE, suI,
                      suD, down, sdE, sdD, sdI, weights, w_dtype, sel, out, bad_index, ws,
                      BIOPS_MOE_NOALLOC_SCRATCH_BYTES, s);
  if (order) {
    // recorded even after a failed launch, so that a later call never waits on work that
    // was not queued
    const hipError_t e = hipEventRecord(o.done, s);
    if (e != hipSuccess && rc == BIOPS_OK) return fail(BIOPS_ERR_HIP, "hipEventRecord: %s", hipGetErrorString(e));
    o.recorded = o.recorded || e == hipSuccess;
  }
  return rc;
}
