// Precompiled CDNA4 kernels for every plan instruction that is not a fused group or a product:
// single elementwise operations, structural copies, int32 gather/scatter, RNG, casts, argmax,
// sort and scan, reductions, and the helpers of the device-resident step loop.
//
// All of these are HBM-bound: wave64 blocks of 256 threads, coalesced row-major access, no LDS
// except where a reduction combines partial results.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <type_traits>

#include "kernels.h"
#include "ops.h"

namespace rgk {

namespace {

constexpr int TPB = 256;

inline uint32_t blocks_for(uint64_t n, uint64_t per_block) { return (uint32_t)((n + per_block - 1) / per_block); }

template <class T> struct Red;
template <> struct Red<float> {
  static __device__ __forceinline__ float init(int kind) { return kind == RG_REDUCE_SUM ? 0.0f : kind == RG_REDUCE_MAX ? -INFINITY : INFINITY; }
};
template <> struct Red<double> {
  static __device__ __forceinline__ double init(int kind) { return kind == RG_REDUCE_SUM ? 0.0 : kind == RG_REDUCE_MAX ? -INFINITY : INFINITY; }
};

template <class T>
__device__ __forceinline__ T combine(int kind, T acc, T x) {
  return kind == RG_REDUCE_SUM ? acc + x : kind == RG_REDUCE_MAX ? rg_max(acc, x) : rg_min(acc, x);
}

__device__ __forceinline__ void decompose(const Strided& g, uint32_t i, uint32_t* off, int nops) {
  for (int k = 0; k < nops; k++) off[k] = g.base[k];
  for (int d = g.rank - 1; d >= 0; d--) {
    uint32_t q = g.size[d].div(i);
    uint32_t c = i - q * g.size[d].d;
    for (int k = 0; k < nops; k++) off[k] += c * g.st[k][d];
    i = q;
  }
}

// ---- elementwise -------------------------------------------------------------------------

template <class T>
__global__ void __launch_bounds__(TPB) k_unary(int op, const T* __restrict__ a, T* d, uint32_t n) {
  uint32_t i = blockIdx.x * TPB + threadIdx.x;
  if (i < n) d[i] = rg_unary<T>(op, a[i]);
}

// mode: 0 same shape, 1 a is a scalar, 2 b is a scalar (src/plan.rs:1008-1023).
template <class T>
__global__ void __launch_bounds__(TPB) k_binary(int op, const T* a, const T* b, T* d, uint32_t n, int mode) {
  uint32_t i = blockIdx.x * TPB + threadIdx.x;
  if (i >= n) return;
  T x = mode == 1 ? a[0] : a[i];
  T y = mode == 2 ? b[0] : b[i];
  d[i] = rg_binary<T>(op, x, y);
}

template <class T>
__global__ void __launch_bounds__(TPB) k_binary_general(int op, const T* a, const T* b, T* d, uint32_t n, Strided g) {
  uint32_t i = blockIdx.x * TPB + threadIdx.x;
  if (i >= n) return;
  uint32_t off[2];
  decompose(g, i, off, 2);
  d[i] = rg_binary<T>(op, a[off[0]], b[off[1]]);
}

__global__ void __launch_bounds__(TPB) k_binary_int(int op, const int* a, const int* b, int* d, uint32_t n, int mode) {
  uint32_t i = blockIdx.x * TPB + threadIdx.x;
  if (i >= n) return;
  int x = mode == 1 ? a[0] : a[i];
  int y = mode == 2 ? b[0] : b[i];
  d[i] = rg_binary_int(op, x, y);
}

__global__ void __launch_bounds__(TPB) k_binary_int_general(int op, const int* a, const int* b, int* d, uint32_t n, Strided g) {
  uint32_t i = blockIdx.x * TPB + threadIdx.x;
  if (i >= n) return;
  uint32_t off[2];
  decompose(g, i, off, 2);
  d[i] = rg_binary_int(op, a[off[0]], b[off[1]]);
}

template <class T>
__global__ void __launch_bounds__(TPB) k_where(const T* c, const T* a, const T* b, T* d, uint32_t n) {
  uint32_t i = blockIdx.x * TPB + threadIdx.x;
  if (i < n) d[i] = c[i] != (T)0 ? a[i] : b[i];
}

// ---- structural copies (any dtype, moved as 32- or 64-bit words) ------------------------

template <class E>
__global__ void __launch_bounds__(TPB) k_gather(const E* __restrict__ src, E* __restrict__ dst, uint32_t n, Strided g) {
  uint32_t i = blockIdx.x * TPB + threadIdx.x;
  if (i >= n) return;
  uint32_t off[1];
  decompose(g, i, off, 1);
  dst[i] = src[off[0]];
}

// Four consecutive outputs per thread (the innermost merged dim is a multiple of 4, so they
// share every outer coordinate): one 16-byte store, and one 16-byte load when the source run is
// contiguous and aligned, a single broadcast load when its stride is 0.
__global__ void __launch_bounds__(TPB) k_gather4(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst, uint32_t n, Strided g,
                                                 int aligned) {
  uint32_t i0 = (blockIdx.x * TPB + threadIdx.x) * 4;
  if (i0 >= n) return;
  uint32_t off[1];
  decompose(g, i0, off, 1);
  uint32_t s_in = g.rank ? g.st[0][g.rank - 1] : 0;
  uint4 v;
  if (s_in == 1 && aligned) {
    v = *(const uint4*)(src + off[0]);
  } else if (s_in == 0) {
    uint32_t x = src[off[0]];
    v = make_uint4(x, x, x, x);
  } else {
    v = make_uint4(src[off[0]], src[off[0] + s_in], src[off[0] + 2 * s_in], src[off[0] + 3 * s_in]);
  }
  *(uint4*)(dst + i0) = v;
}

struct PadDims {
  int rank;
  FastDiv size[MAX_DIMS];
  uint32_t start[MAX_DIMS], len[MAX_DIMS], src_st[MAX_DIMS];
};

template <class E>
__global__ void __launch_bounds__(TPB) k_pad(const E* __restrict__ src, E* __restrict__ dst, uint32_t n, PadDims p) {
  uint32_t i = blockIdx.x * TPB + threadIdx.x;
  if (i >= n) return;
  uint32_t off = 0, rem = i;
  bool inside = true;
  for (int d = p.rank - 1; d >= 0; d--) {
    uint32_t q = p.size[d].div(rem);
    uint32_t c = rem - q * p.size[d].d;
    rem = q;
    if (c < p.start[d] || c >= p.start[d] + p.len[d]) inside = false;
    else off += (c - p.start[d]) * p.src_st[d];
  }
  dst[i] = inside ? src[off] : (E)0;
}

__global__ void __launch_bounds__(TPB) k_pad4(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst, uint32_t n, PadDims p) {
  uint32_t i0 = (blockIdx.x * TPB + threadIdx.x) * 4;
  if (i0 >= n) return;
  uint32_t off = 0, rem = i0;
  bool inside = true;
  for (int d = p.rank - 1; d >= 0; d--) {
    uint32_t q = p.size[d].div(rem);
    uint32_t c = rem - q * p.size[d].d;
    rem = q;
    if (c < p.start[d] || c >= p.start[d] + p.len[d]) inside = false;
    else off += (c - p.start[d]) * p.src_st[d];
  }
  *(uint4*)(dst + i0) = inside ? *(const uint4*)(src + off) : make_uint4(0, 0, 0, 0);
}

template <class E>
__global__ void __launch_bounds__(TPB) k_concat_piece(const E* __restrict__ src, E* __restrict__ dst, uint32_t n, FastDiv len,
                                                      uint32_t total, uint32_t at) {
  uint32_t i = blockIdx.x * TPB + threadIdx.x;
  if (i >= n) return;
  uint32_t o = len.div(i);
  uint32_t q = i - o * len.d;
  dst[o * total + at + q] = src[i];
}

__device__ __forceinline__ uint32_t clamp_index(int ix, uint32_t dim) { return ix < 0 ? 0u : ((uint32_t)ix >= dim ? dim - 1 : (uint32_t)ix); }

template <class E>
__global__ void __launch_bounds__(TPB) k_take(const E* __restrict__ src, const int* __restrict__ idx, E* __restrict__ dst, uint32_t n,
                                              FastDiv block, FastDiv n_idx, uint32_t dim) {
  uint32_t t = blockIdx.x * TPB + threadIdx.x;
  if (t >= n) return;
  uint32_t r = block.div(t);
  uint32_t q = t - r * block.d;
  uint32_t o = n_idx.div(r);
  uint32_t j = r - o * n_idx.d;
  dst[t] = src[(o * dim + clamp_index(idx[j], dim)) * block.d + q];
}

// The same gather, 16 bytes per thread, for rows whose length in bytes is a multiple of 16 (the
// rows then start 16-byte aligned in 256-byte aligned slots): `block` and positions count vectors.
__global__ void __launch_bounds__(TPB) k_take16(const uint4* __restrict__ src, const int* __restrict__ idx, uint4* __restrict__ dst,
                                                uint32_t n, FastDiv block, FastDiv n_idx, uint32_t dim) {
  uint32_t t = blockIdx.x * TPB + threadIdx.x;
  if (t >= n) return;
  uint32_t r = block.div(t);
  uint32_t q = t - r * block.d;
  uint32_t o = n_idx.div(r);
  uint32_t j = r - o * n_idx.d;
  dst[t] = src[(o * dim + clamp_index(idx[j], dim)) * block.d + q];
}

template <class E>
__global__ void __launch_bounds__(TPB) k_take_along(const E* __restrict__ src, const int* __restrict__ idx, E* __restrict__ dst,
                                                    uint32_t n, FastDiv k, uint32_t v) {
  uint32_t j = blockIdx.x * TPB + threadIdx.x;
  if (j >= n) return;
  dst[j] = src[k.div(j) * v + clamp_index(idx[j], v)];
}

// ---- deterministic scatter-add ------------------------------------------------------------
// Each output element sums the cotangents whose index hits it, in increasing index position:
// the CPU's sequential order (src/plan.rs:1502-1531), so results are bit-identical. Index chunks
// are staged in LDS and shared by the block.

constexpr uint32_t TG_PER = 32;                // index entries each thread classifies per chunk
constexpr uint32_t TG_CHUNK = TPB * TG_PER;     // 8192 entries: 32 KB of positions in LDS

// Block (x, d, o) owns columns [x*256, x*256+256) of output row (o, d). Per chunk of 8192 index
// entries, each thread classifies 32 consecutive entries (a bit mask of those that hit row d),
// a block-wide exclusive scan of the mask counts places the matching positions in LDS in
// increasing order, and every thread then sums its column over that list: the CPU's order, with
// coalesced row reads. The adds are sequential but the loads are not: TG_INFLIGHT rows are loaded
// before the first of them is added, so a row hit ~100 times costs a few memory latencies.
template <class T>
__global__ void __launch_bounds__(TPB) k_take_grad(const T* __restrict__ ct, const int* __restrict__ idx, T* __restrict__ dst,
                                                   uint32_t block, uint32_t dim, uint32_t n_idx) {
  constexpr uint32_t TG_INFLIGHT = sizeof(T) == 4 ? 64 : 32;
  __shared__ uint32_t list[TG_CHUNK];
  __shared__ uint32_t wave_total[TPB / 64];
  const uint32_t d = blockIdx.y, o = blockIdx.z;
  const uint32_t q = blockIdx.x * TPB + threadIdx.x;
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const bool vec = ((uintptr_t)idx & 15u) == 0;
  const T* base = ct + (uint64_t)o * n_idx * block + (q < block ? q : 0);
  T acc = (T)0;
  for (uint32_t j0 = 0; j0 < n_idx; j0 += TG_CHUNK) {
    const uint32_t m = min(TG_CHUNK, n_idx - j0);
    const uint32_t lo = threadIdx.x * TG_PER;
    uint32_t bits = 0;
    if (vec && lo + TG_PER <= m) {
      const int4* p = reinterpret_cast<const int4*>(idx + j0 + lo);
#pragma unroll
      for (uint32_t u = 0; u < TG_PER / 4; u++) {
        const int4 w = p[u];
        bits |= (uint32_t)(clamp_index(w.x, dim) == d) << (4 * u);
        bits |= (uint32_t)(clamp_index(w.y, dim) == d) << (4 * u + 1);
        bits |= (uint32_t)(clamp_index(w.z, dim) == d) << (4 * u + 2);
        bits |= (uint32_t)(clamp_index(w.w, dim) == d) << (4 * u + 3);
      }
    } else {
      for (uint32_t u = 0; u < TG_PER && lo + u < m; u++) bits |= (uint32_t)(clamp_index(idx[j0 + lo + u], dim) == d) << u;
    }
    // Exclusive scan of the per-thread counts: within the wave by shuffles, across waves by LDS.
    const uint32_t c = __popc(bits);
    uint32_t incl = c;
#pragma unroll
    for (uint32_t off = 1; off < 64; off <<= 1) {
      const uint32_t v = __shfl_up(incl, off, 64);
      if (lane >= off) incl += v;
    }
    if (lane == 63) wave_total[wave] = incl;
    __syncthreads();
    uint32_t at = incl - c, len = 0;
#pragma unroll
    for (uint32_t w = 0; w < TPB / 64; w++) {
      const uint32_t t = wave_total[w];
      at += w < wave ? t : 0u;
      len += t;
    }
    while (bits) {
      const uint32_t u = __ffs(bits) - 1;
      bits &= bits - 1;
      list[at++] = j0 + lo + u;
    }
    __syncthreads();
    if (q < block) {
      uint32_t e = 0;
      for (; e + TG_INFLIGHT <= len; e += TG_INFLIGHT) {
        T v[TG_INFLIGHT];
#pragma unroll
        for (uint32_t u = 0; u < TG_INFLIGHT; u++) v[u] = base[(uint64_t)list[e + u] * block];
#pragma unroll
        for (uint32_t u = 0; u < TG_INFLIGHT; u++) acc = acc + v[u];
      }
      for (; e + 8 <= len; e += 8) {
        T v[8];
#pragma unroll
        for (uint32_t u = 0; u < 8; u++) v[u] = base[(uint64_t)list[e + u] * block];
#pragma unroll
        for (uint32_t u = 0; u < 8; u++) acc = acc + v[u];
      }
      for (; e < len; e++) acc = acc + base[(uint64_t)list[e] * block];
    }
    __syncthreads();
  }
  if (q < block) dst[((uint64_t)o * dim + d) * block + q] = acc;
}

template <class T>
__global__ void __launch_bounds__(TPB) k_take_along_grad(const T* __restrict__ ct, const int* __restrict__ idx, T* __restrict__ dst,
                                                         uint32_t n, FastDiv v, uint32_t k) {
  uint32_t t = blockIdx.x * TPB + threadIdx.x;
  if (t >= n) return;
  uint32_t r = v.div(t);
  uint32_t c = t - r * v.d;
  T acc = (T)0;
  for (uint32_t x = 0; x < k; x++)
    if (clamp_index(idx[r * k + x], v.d) == c) acc = acc + ct[r * k + x];
  dst[t] = acc;
}

// ---- random streams (SplitMix64 of key and index, src/plan.rs:1391-1435) ----------------

constexpr uint64_t GAMMA = 0x9E3779B97F4A7C15ull;
constexpr uint64_t GAMMA_SPLIT = 0xD1B54A32D192ED03ull;

__device__ __forceinline__ uint64_t mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t read_key(const int* k) { return ((uint64_t)(uint32_t)k[0] << 32) | (uint64_t)(uint32_t)k[1]; }

template <class T>
__global__ void __launch_bounds__(TPB) k_rand_uniform(const int* __restrict__ key, T* __restrict__ dst, uint32_t n) {
  uint32_t j = blockIdx.x * TPB + threadIdx.x;
  if (j >= n) return;
  uint64_t kk = read_key(key);
  constexpr int mant = sizeof(T) == 4 ? 24 : 53;
  uint64_t bits = mix(kk + ((uint64_t)j + 1) * GAMMA) >> (64 - mant);
  dst[j] = (T)((double)bits * (1.0 / (double)(1ull << mant)));
}

template <class T>
__global__ void __launch_bounds__(TPB) k_rand_normal(const int* __restrict__ key, T* __restrict__ dst, uint32_t n) {
  uint32_t j = blockIdx.x * TPB + threadIdx.x;
  if (j >= n) return;
  uint64_t kk = read_key(key);
  const double scale = 1.0 / 9007199254740992.0;  // 2^-53
  double u1 = 1.0 - (double)(mix(kk + (2 * (uint64_t)j + 1) * GAMMA) >> 11) * scale;
  double u2 = (double)(mix(kk + (2 * (uint64_t)j + 2) * GAMMA) >> 11) * scale;
  dst[j] = (T)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}

__global__ void __launch_bounds__(TPB) k_key_split(const int* __restrict__ key, int* __restrict__ dst, uint32_t pairs) {
  uint32_t j = blockIdx.x * TPB + threadIdx.x;
  if (j >= pairs) return;
  uint64_t bits = mix(read_key(key) + ((uint64_t)j + 1) * GAMMA_SPLIT);
  dst[2 * j] = (int)(uint32_t)(bits >> 32);
  dst[2 * j + 1] = (int)(uint32_t)bits;
}

// ---- casts (Rust `as`: float to int truncates, saturates, NaN is 0) ---------------------

__device__ __forceinline__ int sat_i32(double x) {
  if (x != x) return 0;
  if (x >= 2147483647.0) return 2147483647;
  if (x <= -2147483648.0) return (int)0x80000000u;
  return (int)x;
}

template <class S, class D>
__global__ void __launch_bounds__(TPB) k_cast(const S* __restrict__ a, D* __restrict__ d, uint32_t n) {
  uint32_t i = blockIdx.x * TPB + threadIdx.x;
  if (i >= n) return;
  if constexpr (sizeof(D) == 4 && !std::is_floating_point<D>::value) d[i] = sat_i32((double)a[i]);
  else d[i] = (D)a[i];
}

// ---- argmax, top-k, cumsum (one row per thread, in the CPU's order) --------------------

template <class T>
__global__ void __launch_bounds__(TPB) k_argmax(const T* __restrict__ a, int* __restrict__ d, uint32_t rows, uint32_t v) {
  uint32_t r = blockIdx.x * TPB + threadIdx.x;
  if (r >= rows) return;
  const T* row = a + (uint64_t)r * v;
  uint32_t best = 0;
  for (uint32_t j = 0; j < v; j++)
    if (row[j] > row[best]) best = j;
  d[r] = (int)best;
}

// Ranking of src/plan.rs:838-848: a value ranks ahead when greater, or equal with a lower position; NaN ranks behind all.
template <class T>
__device__ __forceinline__ bool before(const T* row, uint32_t x, uint32_t y) {
  T p = row[x], q = row[y];
  bool pn = p != p, qn = q != q;
  if (pn || qn) return pn != qn ? qn : x < y;
  if (p != q) return p > q;
  return x < y;
}

// The same ranking by value: p at position x ahead of q at position y.
template <class T>
__device__ __forceinline__ bool before_v(T p, uint32_t x, T q, uint32_t y) {
  bool pn = p != p, qn = q != q;
  if (pn || qn) return pn != qn ? qn : x < y;
  if (p != q) return p > q;
  return x < y;
}

// Rows of at most TOPK_RANK_MAX values: one block per row, the row in LDS, and every position's
// rank (the number of positions ranking ahead of it) counted in parallel; positions ranked below
// k are written at their rank. The ranking is a strict total order, so this is the same output
// as choosing each next position in turn (k_arg_top_k below, for longer rows).
constexpr uint32_t TOPK_RANK_MAX = 4096;
template <class T>
__global__ void __launch_bounds__(256) k_arg_top_k_rank(const T* __restrict__ a, int* __restrict__ d, uint32_t v, uint32_t k) {
  __shared__ T vals[TOPK_RANK_MAX];
  const uint64_t r = blockIdx.x;
  const T* row = a + r * v;
  for (uint32_t j = threadIdx.x; j < v; j += 256) vals[j] = row[j];
  __syncthreads();
  for (uint32_t j = threadIdx.x; j < v; j += 256) {
    const T q = vals[j];
    uint32_t rank = 0;
    for (uint32_t i = 0; i < v; i++) rank += before_v(vals[i], i, q, j) ? 1u : 0u;
    if (rank < k) d[r * k + rank] = (int)j;
  }
}

template <class T>
__global__ void __launch_bounds__(TPB) k_arg_top_k(const T* __restrict__ a, int* __restrict__ d, uint32_t rows, uint32_t v, uint32_t k) {
  uint32_t r = blockIdx.x * TPB + threadIdx.x;
  if (r >= rows) return;
  const T* row = a + (uint64_t)r * v;
  // Each output is the successor of the previous one in the total order.
  uint32_t prev = 0;
  for (uint32_t p = 0; p < k; p++) {
    uint32_t best = 0xffffffffu;
    for (uint32_t j = 0; j < v; j++) {
      if (p > 0 && !before(row, prev, j)) continue;
      if (best == 0xffffffffu || before(row, j, best)) best = j;
    }
    d[(uint64_t)r * k + p] = (int)best;
    prev = best;
  }
}

template <class T>
__global__ void __launch_bounds__(TPB) k_cumsum(const T* __restrict__ a, T* __restrict__ d, uint32_t rows, uint32_t v, int reverse) {
  uint32_t r = blockIdx.x * TPB + threadIdx.x;
  if (r >= rows) return;
  const T* x = a + (uint64_t)r * v;
  T* y = d + (uint64_t)r * v;
  T acc = (T)0;
  if (reverse)
    for (uint32_t j = v; j-- > 0;) y[j] = acc = acc + x[j];
  else
    for (uint32_t j = 0; j < v; j++) y[j] = acc = acc + x[j];
}

__global__ void __launch_bounds__(TPB) k_cumsum_int(const int* __restrict__ a, int* __restrict__ d, uint32_t rows, uint32_t v, int reverse) {
  uint32_t r = blockIdx.x * TPB + threadIdx.x;
  if (r >= rows) return;
  const int* x = a + (uint64_t)r * v;
  int* y = d + (uint64_t)r * v;
  uint32_t acc = 0;
  if (reverse)
    for (uint32_t j = v; j-- > 0;) y[j] = (int)(acc += (uint32_t)x[j]);
  else
    for (uint32_t j = 0; j < v; j++) y[j] = (int)(acc += (uint32_t)x[j]);
}

// ---- reductions ---------------------------------------------------------------------------

template <int KIND, class T>
__device__ __forceinline__ T wave_combine(T v) {
  return rg_wave_all(v, [](T x, T y) { return combine(KIND, x, y); });
}

// One wave per row: rows up to a few thousand elements (LayerNorm, softmax, cross-entropy).
// KIND is a template argument so the combine step has no branch between the loads.
template <class T, int KIND>
__global__ void __launch_bounds__(TPB) k_reduce_rows_wave(const T* __restrict__ a, T* __restrict__ d, uint32_t rows, uint32_t len) {
  uint32_t row = blockIdx.x * (TPB / 64) + threadIdx.x / 64;
  uint32_t lane = threadIdx.x % 64;
  if (row >= rows) return;
  const T* x = a + (uint64_t)row * len;
  T acc = Red<T>::init(KIND);
  constexpr uint32_t V = 16 / sizeof(T);
  if (len % V == 0) {
    // 16-byte loads: lane l reads elements [V*l, V*l+V) of each 64*V segment.
    typedef T vec __attribute__((ext_vector_type(V)));
    for (uint32_t j = lane * V; j < len; j += 64 * V) {
      vec v = *(const vec*)(x + j);
#pragma unroll
      for (uint32_t q = 0; q < V; q++) acc = combine(KIND, acc, v[q]);
    }
  } else {
    for (uint32_t j = lane; j < len; j += 64) acc = combine(KIND, acc, x[j]);
  }
  acc = wave_combine<KIND>(acc);
  if (lane == 0) d[row] = acc;
}

template <class T, int KIND>
__global__ void __launch_bounds__(TPB) k_reduce_rows_block(const T* __restrict__ a, T* __restrict__ d, uint64_t len, uint64_t seg) {
  __shared__ T part[TPB / 64];
  uint64_t row = blockIdx.y;
  uint64_t begin = (uint64_t)blockIdx.x * seg, end = min(len, begin + seg);
  const T* x = a + row * len;
  T acc = Red<T>::init(KIND);
  for (uint64_t j = begin + threadIdx.x; j < end; j += TPB) acc = combine(KIND, acc, x[j]);
  acc = wave_combine<KIND>(acc);
  if (threadIdx.x % 64 == 0) part[threadIdx.x / 64] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    T r = part[0];
    for (int w = 1; w < TPB / 64; w++) r = combine(KIND, r, part[w]);
    d[row * gridDim.x + blockIdx.x] = r;
  }
}

// Leading-axis reduction of [batch, r, k] over r. A block owns 64 consecutive columns (one
// coalesced 256-byte row segment per wave) and LANES row lanes; row chunks give parallelism and
// write partial results, which a second pass of the same kernel combines (deterministic order).
template <class T, int LANES, int KIND>
__global__ void __launch_bounds__(64 * LANES) k_reduce_cols(const T* __restrict__ a, T* __restrict__ out, uint32_t r, uint32_t k,
                                                             uint32_t chunk_rows, uint32_t chunks) {
  __shared__ T part[LANES][64];
  const uint32_t tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const uint32_t c = blockIdx.x * 64 + tx;
  const uint32_t b = blockIdx.y, s = blockIdx.z;
  const uint32_t r0 = s * chunk_rows, r1 = min(r, r0 + chunk_rows);
  T acc = Red<T>::init(KIND);
  if (c < k) {
    // Eight loads in flight per lane, then combined in row order.
    const T* x = a + (uint64_t)b * r * k + c;
    uint32_t row = r0 + ty;
    for (; row + 7 * LANES < r1; row += 8 * LANES) {
      T v[8];
#pragma unroll
      for (int q = 0; q < 8; q++) v[q] = x[(uint64_t)(row + q * LANES) * k];
#pragma unroll
      for (int q = 0; q < 8; q++) acc = combine(KIND, acc, v[q]);
    }
    for (; row < r1; row += LANES) acc = combine(KIND, acc, x[(uint64_t)row * k]);
  }
  part[ty][tx] = acc;
  __syncthreads();
  if (ty == 0 && c < k) {
    T v = part[0][tx];
#pragma unroll
    for (int l = 1; l < LANES; l++) v = combine(KIND, v, part[l][tx]);
    out[((uint64_t)b * chunks + s) * k + c] = v;
  }
}

// The same reduction with 16-byte loads: a lane owns V = 16 / sizeof(T) adjacent columns, so one
// wave covers 64 * V columns (a 1 KiB row segment) and four waves are the row lanes. Eight row
// loads in flight per lane; per column the rows are combined in the same lane-strided order as
// k_reduce_cols. Needs k % V == 0 and a 16-byte aligned base.
template <class T, int KIND>
__global__ void __launch_bounds__(256) k_reduce_cols_vec(const T* __restrict__ a, T* __restrict__ out, uint32_t r, uint32_t k,
                                                         uint32_t chunk_rows, uint32_t chunks) {
  constexpr int V = 16 / sizeof(T), LANES = 4;
  using Vec = T __attribute__((ext_vector_type(V)));
  __shared__ T part[LANES][64 * V];
  const uint32_t tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const uint32_t c = (blockIdx.x * 64 + tx) * V;
  const uint32_t b = blockIdx.y, s = blockIdx.z;
  const uint32_t r0 = s * chunk_rows, r1 = min(r, r0 + chunk_rows);
  Vec acc;
#pragma unroll
  for (int e = 0; e < V; e++) acc[e] = Red<T>::init(KIND);
  if (c < k) {
    const T* x = a + (uint64_t)b * r * k + c;
    uint32_t row = r0 + ty;
    for (; row + 7 * LANES < r1; row += 8 * LANES) {
      Vec v[8];
#pragma unroll
      for (int q = 0; q < 8; q++) v[q] = *(const Vec*)(x + (uint64_t)(row + q * LANES) * k);
#pragma unroll
      for (int q = 0; q < 8; q++)
#pragma unroll
        for (int e = 0; e < V; e++) acc[e] = combine(KIND, acc[e], v[q][e]);
    }
    for (; row < r1; row += LANES) {
      Vec v = *(const Vec*)(x + (uint64_t)row * k);
#pragma unroll
      for (int e = 0; e < V; e++) acc[e] = combine(KIND, acc[e], v[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < V; e++) part[ty][tx * V + e] = acc[e];
  __syncthreads();
  // Each thread finishes 64 * V / 256 columns of the block's tile.
  for (uint32_t j = threadIdx.x; j < 64 * V; j += 256) {
    const uint32_t col = blockIdx.x * 64 * V + j;
    if (col >= k) continue;
    T v = part[0][j];
#pragma unroll
    for (int l = 1; l < LANES; l++) v = combine(KIND, v, part[l][j]);
    out[((uint64_t)b * chunks + s) * k + col] = v;
  }
}

template <class T, int KIND>
__global__ void __launch_bounds__(TPB) k_reduce_general(const T* __restrict__ a, T* __restrict__ d, uint32_t out_n, Strided outer,
                                                        Strided inner, uint32_t red_n) {
  uint32_t o = blockIdx.x * TPB + threadIdx.x;
  if (o >= out_n) return;
  uint32_t base[1];
  decompose(outer, o, base, 1);
  T acc = Red<T>::init(KIND);
  uint32_t r = 0;
  for (; r + 4 <= red_n; r += 4) {  // four loads in flight, combined in order
    T v[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      uint32_t off[1];
      decompose(inner, r + q, off, 1);
      v[q] = a[base[0] + off[0]];
    }
#pragma unroll
    for (int q = 0; q < 4; q++) acc = combine(KIND, acc, v[q]);
  }
  for (; r < red_n; r++) {
    uint32_t off[1];
    decompose(inner, r, off, 1);
    acc = combine(KIND, acc, a[base[0] + off[0]]);
  }
  d[o] = acc;
}

// ---- step-loop helpers ------------------------------------------------------------------

__global__ void __launch_bounds__(TPB) k_copy_words(uint32_t* __restrict__ dst, const uint32_t* __restrict__ src, uint64_t words) {
  uint64_t i = (uint64_t)blockIdx.x * TPB + threadIdx.x;
  if (i < words) dst[i] = src[i];
}

__global__ void k_record_history(int dtype, const void* slot, double* hist, const uint64_t* counter, uint64_t stride) {
  double v = dtype == RG_F32 ? (double)((const float*)slot)[0] : dtype == RG_F64 ? ((const double*)slot)[0] : (double)((const int*)slot)[0];
  hist[*counter % stride] = v;
}

__global__ void __launch_bounds__(TPB) k_load_batch(uint32_t* __restrict__ dst, const uint32_t* __restrict__ batches, uint64_t words,
                                                     uint64_t n_batches, const uint64_t* counter) {
  uint64_t i = (uint64_t)blockIdx.x * TPB + threadIdx.x;
  if (i >= words) return;
  uint64_t b = *counter % n_batches;
  dst[i] = batches[b * words + i];
}

__global__ void k_counter_inc(uint64_t* counter) { *counter += 1; }

__global__ void k_set_counter(uint64_t* counter, uint64_t value) { *counter = value; }

// One thread waits until `ticks` of the constant-rate wall clock have passed: a bounded wait
// that every launch leaves, used to hold a stream while the host enqueues timed work.
__global__ void k_hold(uint64_t ticks) {
  uint64_t t0 = wall_clock64();
  while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(8);
}

__global__ void __launch_bounds__(TPB) k_fill_zero(uint32_t* dst, uint64_t words) {
  uint64_t i = (uint64_t)blockIdx.x * TPB + threadIdx.x;
  if (i < words) dst[i] = 0;
}

}  // namespace

// ---- host side --------------------------------------------------------------------------

std::vector<int64_t> row_strides(const std::vector<int64_t>& shape) {
  std::vector<int64_t> st(shape.size(), 1);
  for (size_t i = shape.size(); i-- > 1;) st[i - 1] = st[i] * shape[i];
  return st;
}

std::vector<int64_t> bcast_strides(const std::vector<int64_t>& shape, size_t rank) {
  auto st = row_strides(shape);
  size_t lead = rank - shape.size();
  std::vector<int64_t> out(rank, 0);
  for (size_t i = 0; i < rank; i++) out[i] = (i < lead || shape[i - lead] == 1) ? 0 : st[i - lead];
  return out;
}

Strided make_strided(const std::vector<int64_t>& shape, const std::vector<std::vector<int64_t>>& strides) {
  size_t nops = strides.size();
  std::vector<int64_t> sz;
  std::vector<std::vector<int64_t>> st(nops);
  for (size_t d = 0; d < shape.size(); d++) {
    if (shape[d] == 1) continue;
    if (!sz.empty()) {
      bool merge = true;
      for (size_t k = 0; k < nops; k++)
        if (st[k].back() != strides[k][d] * shape[d]) merge = false;
      if (merge) {
        sz.back() *= shape[d];
        for (size_t k = 0; k < nops; k++) st[k].back() = strides[k][d];
        continue;
      }
    }
    sz.push_back(shape[d]);
    for (size_t k = 0; k < nops; k++) st[k].push_back(strides[k][d]);
  }
  if (sz.size() > (size_t)MAX_DIMS) throw std::runtime_error("too many non-mergeable dimensions for a strided kernel");
  Strided g;
  g.rank = (int)sz.size();
  for (size_t d = 0; d < sz.size(); d++) {
    g.size[d] = FastDiv((uint32_t)sz[d]);
    for (size_t k = 0; k < nops; k++) g.st[k][d] = (uint32_t)st[k][d];
  }
  return g;
}

#define RG_LAUNCH(kernel, n, ...)                                                   \
  do {                                                                              \
    if ((n) > 0) hipLaunchKernelGGL(kernel, dim3(blocks_for((n), TPB)), dim3(TPB), 0, s, __VA_ARGS__); \
  } while (0)

void unary(hipStream_t s, int dtype, int op, const void* a, void* d, uint64_t n) {
  if (dtype == RG_F32) RG_LAUNCH(k_unary<float>, n, op, (const float*)a, (float*)d, (uint32_t)n);
  else RG_LAUNCH(k_unary<double>, n, op, (const double*)a, (double*)d, (uint32_t)n);
}

void binary(hipStream_t s, int dtype, int op, const void* a, const void* b, void* d, uint64_t n, int mode, const Strided* g) {
  if (dtype == RG_I32) {
    if (g) RG_LAUNCH(k_binary_int_general, n, op, (const int*)a, (const int*)b, (int*)d, (uint32_t)n, *g);
    else RG_LAUNCH(k_binary_int, n, op, (const int*)a, (const int*)b, (int*)d, (uint32_t)n, mode);
  } else if (dtype == RG_F32) {
    if (g) RG_LAUNCH(k_binary_general<float>, n, op, (const float*)a, (const float*)b, (float*)d, (uint32_t)n, *g);
    else RG_LAUNCH(k_binary<float>, n, op, (const float*)a, (const float*)b, (float*)d, (uint32_t)n, mode);
  } else {
    if (g) RG_LAUNCH(k_binary_general<double>, n, op, (const double*)a, (const double*)b, (double*)d, (uint32_t)n, *g);
    else RG_LAUNCH(k_binary<double>, n, op, (const double*)a, (const double*)b, (double*)d, (uint32_t)n, mode);
  }
}

void where(hipStream_t s, int esize, const void* c, const void* a, const void* b, void* d, uint64_t n, int dtype) {
  if (dtype == RG_F32) RG_LAUNCH(k_where<float>, n, (const float*)c, (const float*)a, (const float*)b, (float*)d, (uint32_t)n);
  else if (dtype == RG_F64) RG_LAUNCH(k_where<double>, n, (const double*)c, (const double*)a, (const double*)b, (double*)d, (uint32_t)n);
  else RG_LAUNCH(k_where<int>, n, (const int*)c, (const int*)a, (const int*)b, (int*)d, (uint32_t)n);
  (void)esize;
}

void gather(hipStream_t s, int esize, const void* src, void* dst, uint64_t n, const Strided& g) {
  bool vec = esize == 4 && n % 4 == 0 && (g.rank == 0 || g.size[g.rank - 1].d % 4 == 0) && ((uintptr_t)dst & 15) == 0;
  if (vec) {
    // The source run is 16-byte aligned when the base and every outer stride are multiples of 4.
    bool aligned = ((uintptr_t)src & 15) == 0 && g.base[0] % 4 == 0;
    for (int d = 0; d + 1 < g.rank; d++) aligned = aligned && g.st[0][d] % 4 == 0;
    uint64_t n4 = n / 4;
    if (g.rank == 0) aligned = false;
    RG_LAUNCH(k_gather4, n4, (const uint32_t*)src, (uint32_t*)dst, (uint32_t)n, g, (int)aligned);
    return;
  }
  if (esize == 4) RG_LAUNCH(k_gather<uint32_t>, n, (const uint32_t*)src, (uint32_t*)dst, (uint32_t)n, g);
  else RG_LAUNCH(k_gather<uint64_t>, n, (const uint64_t*)src, (uint64_t*)dst, (uint32_t)n, g);
}

void pad(hipStream_t s, int esize, const void* src, void* dst, uint64_t n, const std::vector<int64_t>& out_shape,
         const std::vector<int64_t>& starts, const std::vector<int64_t>& in_shape) {
  if (out_shape.size() > (size_t)MAX_DIMS) throw std::runtime_error("pad rank above 8");
  PadDims p;
  p.rank = (int)out_shape.size();
  auto st = row_strides(in_shape);
  for (size_t d = 0; d < out_shape.size(); d++) {
    p.size[d] = FastDiv((uint32_t)out_shape[d]);
    p.start[d] = (uint32_t)starts[d];
    p.len[d] = (uint32_t)in_shape[d];
    p.src_st[d] = (uint32_t)st[d];
  }
  size_t last = out_shape.size() - 1;
  bool vec = esize == 4 && !out_shape.empty() && starts[last] == 0 && in_shape[last] == out_shape[last] && out_shape[last] % 4 == 0 &&
             ((uintptr_t)src & 15) == 0 && ((uintptr_t)dst & 15) == 0;
  if (vec) {
    RG_LAUNCH(k_pad4, n / 4, (const uint32_t*)src, (uint32_t*)dst, (uint32_t)n, p);
    return;
  }
  if (esize == 4) RG_LAUNCH(k_pad<uint32_t>, n, (const uint32_t*)src, (uint32_t*)dst, (uint32_t)n, p);
  else RG_LAUNCH(k_pad<uint64_t>, n, (const uint64_t*)src, (uint64_t*)dst, (uint32_t)n, p);
}

void concat_piece(hipStream_t s, int esize, const void* src, void* dst, uint64_t outer, uint64_t len, uint64_t total, uint64_t at) {
  uint64_t n = outer * len;
  if (len == 0) return;
  FastDiv l((uint32_t)len);
  if (esize == 4) RG_LAUNCH(k_concat_piece<uint32_t>, n, (const uint32_t*)src, (uint32_t*)dst, (uint32_t)n, l, (uint32_t)total, (uint32_t)at);
  else RG_LAUNCH(k_concat_piece<uint64_t>, n, (const uint64_t*)src, (uint64_t*)dst, (uint32_t)n, l, (uint32_t)total, (uint32_t)at);
}

void take(hipStream_t s, int esize, const void* src, const int32_t* idx, void* dst, uint64_t n, uint64_t block, uint64_t n_idx,
          uint64_t dim) {
  if (n_idx == 0 || block == 0) return;
  if ((block * esize) % 16 == 0 && (uintptr_t)src % 16 == 0 && (uintptr_t)dst % 16 == 0) {
    const uint64_t per = block * esize / 16;  // vectors per row
    FastDiv fb((uint32_t)per), fi((uint32_t)n_idx);
    const uint64_t nv = n * esize / 16;
    RG_LAUNCH(k_take16, nv, (const uint4*)src, idx, (uint4*)dst, (uint32_t)nv, fb, fi, (uint32_t)dim);
    return;
  }
  FastDiv fb((uint32_t)block), fi((uint32_t)n_idx);
  if (esize == 4) RG_LAUNCH(k_take<uint32_t>, n, (const uint32_t*)src, idx, (uint32_t*)dst, (uint32_t)n, fb, fi, (uint32_t)dim);
  else RG_LAUNCH(k_take<uint64_t>, n, (const uint64_t*)src, idx, (uint64_t*)dst, (uint32_t)n, fb, fi, (uint32_t)dim);
}

void take_along(hipStream_t s, int esize, const void* src, const int32_t* idx, void* dst, uint64_t n, uint64_t k, uint64_t v) {
  if (k == 0) return;
  FastDiv fk((uint32_t)k);
  if (esize == 4) RG_LAUNCH(k_take_along<uint32_t>, n, (const uint32_t*)src, idx, (uint32_t*)dst, (uint32_t)n, fk, (uint32_t)v);
  else RG_LAUNCH(k_take_along<uint64_t>, n, (const uint64_t*)src, idx, (uint64_t*)dst, (uint32_t)n, fk, (uint32_t)v);
}

void take_grad(hipStream_t s, int dtype, const void* ct, const int32_t* idx, void* dst, uint64_t n, uint64_t block, uint64_t n_idx,
               uint64_t dim) {
  if (block == 0 || n == 0) return;
  uint64_t outer = n / (block * dim);
  dim3 grid(blocks_for(block, TPB), (uint32_t)dim, (uint32_t)outer);
  if (dtype == RG_F32)
    hipLaunchKernelGGL(k_take_grad<float>, grid, dim3(TPB), 0, s, (const float*)ct, idx, (float*)dst, (uint32_t)block, (uint32_t)dim, (uint32_t)n_idx);
  else
    hipLaunchKernelGGL(k_take_grad<double>, grid, dim3(TPB), 0, s, (const double*)ct, idx, (double*)dst, (uint32_t)block, (uint32_t)dim, (uint32_t)n_idx);
}

void take_along_grad(hipStream_t s, int dtype, const void* ct, const int32_t* idx, void* dst, uint64_t n, uint64_t k, uint64_t v) {
  FastDiv fv((uint32_t)v);
  if (dtype == RG_F32) RG_LAUNCH(k_take_along_grad<float>, n, (const float*)ct, idx, (float*)dst, (uint32_t)n, fv, (uint32_t)k);
  else RG_LAUNCH(k_take_along_grad<double>, n, (const double*)ct, idx, (double*)dst, (uint32_t)n, fv, (uint32_t)k);
}

void rand_uniform(hipStream_t s, int dtype, const int32_t* key, void* dst, uint64_t n) {
  if (dtype == RG_F32) RG_LAUNCH(k_rand_uniform<float>, n, key, (float*)dst, (uint32_t)n);
  else RG_LAUNCH(k_rand_uniform<double>, n, key, (double*)dst, (uint32_t)n);
}

void rand_normal(hipStream_t s, int dtype, const int32_t* key, void* dst, uint64_t n) {
  if (dtype == RG_F32) RG_LAUNCH(k_rand_normal<float>, n, key, (float*)dst, (uint32_t)n);
  else RG_LAUNCH(k_rand_normal<double>, n, key, (double*)dst, (uint32_t)n);
}

void key_split(hipStream_t s, const int32_t* key, int32_t* dst, uint64_t pairs) { RG_LAUNCH(k_key_split, pairs, key, dst, (uint32_t)pairs); }

void cast(hipStream_t s, int from, int to, const void* a, void* d, uint64_t n) {
#define RG_CAST(S, D) RG_LAUNCH((k_cast<S, D>), n, (const S*)a, (D*)d, (uint32_t)n)
  if (from == RG_F32 && to == RG_F64) RG_CAST(float, double);
  else if (from == RG_F32 && to == RG_I32) RG_CAST(float, int);
  else if (from == RG_F64 && to == RG_F32) RG_CAST(double, float);
  else if (from == RG_F64 && to == RG_I32) RG_CAST(double, int);
  else if (from == RG_I32 && to == RG_F32) RG_CAST(int, float);
  else if (from == RG_I32 && to == RG_F64) RG_CAST(int, double);
  else hipMemcpyAsync(d, a, n * (from == RG_F64 ? 8 : 4), hipMemcpyDeviceToDevice, s);
#undef RG_CAST
}

void argmax(hipStream_t s, int dtype, const void* a, int32_t* d, uint64_t rows, uint64_t v) {
  if (dtype == RG_F32) RG_LAUNCH(k_argmax<float>, rows, (const float*)a, d, (uint32_t)rows, (uint32_t)v);
  else RG_LAUNCH(k_argmax<double>, rows, (const double*)a, d, (uint32_t)rows, (uint32_t)v);
}

void arg_top_k(hipStream_t s, int dtype, const void* a, int32_t* d, uint64_t rows, uint64_t v, uint64_t k) {
  if (rows == 0 || k == 0) return;
  // Rough latencies in dependent steps: choosing in turn walks k * v cached global reads per row,
  // every row at once; ranking walks v * ceil(v / 256) LDS reads (about 20 times cheaper), about
  // 2048 rows (blocks) at a time. Many long rows with a small k stay on the first.
  const uint64_t turn = ((rows + 65535) / 65536) * k * v;
  const uint64_t rank = ((rows + 2047) / 2048) * v * ((v + 255) / 256) / 20;
  if (v <= TOPK_RANK_MAX && rank <= turn) {
    if (dtype == RG_F32) hipLaunchKernelGGL(k_arg_top_k_rank<float>, dim3((uint32_t)rows), dim3(256), 0, s, (const float*)a, d, (uint32_t)v, (uint32_t)k);
    else hipLaunchKernelGGL(k_arg_top_k_rank<double>, dim3((uint32_t)rows), dim3(256), 0, s, (const double*)a, d, (uint32_t)v, (uint32_t)k);
    return;
  }
  if (dtype == RG_F32) RG_LAUNCH(k_arg_top_k<float>, rows, (const float*)a, d, (uint32_t)rows, (uint32_t)v, (uint32_t)k);
  else RG_LAUNCH(k_arg_top_k<double>, rows, (const double*)a, d, (uint32_t)rows, (uint32_t)v, (uint32_t)k);
}

void cumsum(hipStream_t s, int dtype, const void* a, void* d, uint64_t rows, uint64_t v, bool reverse) {
  if (dtype == RG_F32) RG_LAUNCH(k_cumsum<float>, rows, (const float*)a, (float*)d, (uint32_t)rows, (uint32_t)v, (int)reverse);
  else if (dtype == RG_F64) RG_LAUNCH(k_cumsum<double>, rows, (const double*)a, (double*)d, (uint32_t)rows, (uint32_t)v, (int)reverse);
  else RG_LAUNCH(k_cumsum_int, rows, (const int*)a, (int*)d, (uint32_t)rows, (uint32_t)v, (int)reverse);
}

// Calls F with the reduction kind as a compile-time constant.
template <class F>
void with_kind(int kind, F f) {
  if (kind == RG_REDUCE_SUM) f(std::integral_constant<int, RG_REDUCE_SUM>());
  else if (kind == RG_REDUCE_MAX) f(std::integral_constant<int, RG_REDUCE_MAX>());
  else f(std::integral_constant<int, RG_REDUCE_MIN>());
}

void reduce_rows(hipStream_t s, int dtype, int kind, const void* a, void* d, uint64_t rows, uint64_t len) {
  if (rows == 0) return;
  with_kind(kind, [&](auto K) {
    constexpr int KIND = decltype(K)::value;
    if (len <= 4096) {
      uint32_t grid = blocks_for(rows, TPB / 64);
      if (dtype == RG_F32) hipLaunchKernelGGL((k_reduce_rows_wave<float, KIND>), dim3(grid), dim3(TPB), 0, s, (const float*)a, (float*)d, (uint32_t)rows, (uint32_t)len);
      else hipLaunchKernelGGL((k_reduce_rows_wave<double, KIND>), dim3(grid), dim3(TPB), 0, s, (const double*)a, (double*)d, (uint32_t)rows, (uint32_t)len);
    } else {
      if (dtype == RG_F32) hipLaunchKernelGGL((k_reduce_rows_block<float, KIND>), dim3(1, (uint32_t)rows), dim3(TPB), 0, s, (const float*)a, (float*)d, len, len);
      else hipLaunchKernelGGL((k_reduce_rows_block<double, KIND>), dim3(1, (uint32_t)rows), dim3(TPB), 0, s, (const double*)a, (double*)d, len, len);
    }
  });
}

static bool reduce_cols_vector(int dtype, const void* a, uint64_t k) {
  const uint64_t v = dtype == RG_F32 ? 4 : 2;
  return k % v == 0 && ((uintptr_t)a & 15) == 0;
}

uint64_t reduce_cols_chunks(int dtype, uint64_t batch, uint64_t r, uint64_t k) {
  // About 512 blocks in the first pass (2 per CU), at least 32 rows per chunk (one round of eight
  // loads per row lane), and at most 256 chunks so the combining pass stays one round of loads per
  // thread. The column tile is 64 lanes of 16 bytes when k allows vector loads, else 64 columns.
  const uint64_t tile = k % (dtype == RG_F32 ? 4 : 2) == 0 ? (dtype == RG_F32 ? 256 : 128) : 64;
  uint64_t col_blocks = (k + tile - 1) / tile * batch;
  uint64_t want = (512 + col_blocks - 1) / col_blocks;
  uint64_t chunks = std::max<uint64_t>(1, std::min<uint64_t>(want, r / 32));
  return std::min<uint64_t>(chunks, 256);
}

void reduce_cols(hipStream_t s, int dtype, int kind, const void* a, void* d, uint64_t batch, uint64_t r, uint64_t k, void* partial,
                 uint64_t chunks) {
  uint32_t chunk_rows = (uint32_t)((r + chunks - 1) / chunks);
  void* out = chunks == 1 ? d : partial;
  const bool vec = reduce_cols_vector(dtype, a, k);
  with_kind(kind, [&](auto K) {
    constexpr int KIND = decltype(K)::value;
    if (vec) {
      dim3 grid(blocks_for(k, dtype == RG_F32 ? 256 : 128), (uint32_t)batch, (uint32_t)chunks);
      if (dtype == RG_F32)
        hipLaunchKernelGGL((k_reduce_cols_vec<float, KIND>), grid, dim3(256), 0, s, (const float*)a, (float*)out, (uint32_t)r,
                           (uint32_t)k, chunk_rows, (uint32_t)chunks);
      else
        hipLaunchKernelGGL((k_reduce_cols_vec<double, KIND>), grid, dim3(256), 0, s, (const double*)a, (double*)out, (uint32_t)r,
                           (uint32_t)k, chunk_rows, (uint32_t)chunks);
    } else {
      dim3 grid(blocks_for(k, 64), (uint32_t)batch, (uint32_t)chunks);
      if (dtype == RG_F32)
        hipLaunchKernelGGL((k_reduce_cols<float, 4, KIND>), grid, dim3(256), 0, s, (const float*)a, (float*)out, (uint32_t)r, (uint32_t)k,
                           chunk_rows, (uint32_t)chunks);
      else
        hipLaunchKernelGGL((k_reduce_cols<double, 4, KIND>), grid, dim3(256), 0, s, (const double*)a, (double*)out, (uint32_t)r, (uint32_t)k,
                           chunk_rows, (uint32_t)chunks);
    }
    if (chunks > 1 && d != nullptr) {
      // The partials [batch, chunks, k] are themselves a leading-axis reduction: 16 row lanes.
      dim3 g2(blocks_for(k, 64), (uint32_t)batch, 1);
      if (dtype == RG_F32)
        hipLaunchKernelGGL((k_reduce_cols<float, 16, KIND>), g2, dim3(1024), 0, s, (const float*)partial, (float*)d, (uint32_t)chunks,
                           (uint32_t)k, (uint32_t)chunks, 1u);
      else
        hipLaunchKernelGGL((k_reduce_cols<double, 16, KIND>), g2, dim3(1024), 0, s, (const double*)partial, (double*)d, (uint32_t)chunks,
                           (uint32_t)k, (uint32_t)chunks, 1u);
    }
  });
}

// Several f32 folds in one launch: block b folds 64 columns of the job whose column tiles it
// falls in, 16 row lanes each folding a run of rows in order, the lanes then combined in order
// (the same order as k_reduce_cols' combining pass).
__global__ void __launch_bounds__(1024) k_fold_jobs(FoldJobs jobs) {
  __shared__ float part[16][64];
  uint32_t j = 0;
  while (j + 1 < jobs.n && blockIdx.x >= jobs.job[j + 1].first_tile) j++;
  const FoldJob& f = jobs.job[j];
  const uint32_t tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const uint32_t c = (blockIdx.x - f.first_tile) * 64 + tx;
  float acc = Red<float>::init(f.kind);
  if (c < f.k) {
    uint32_t r = ty;
    for (; r + 7 * 16 < f.rows; r += 8 * 16) {
      float v[8];
#pragma unroll
      for (int q = 0; q < 8; q++) v[q] = f.part[(uint64_t)(r + q * 16) * f.k + c];
#pragma unroll
      for (int q = 0; q < 8; q++) acc = combine(f.kind, acc, v[q]);
    }
    if (r < f.rows) {  // the last rows as one guarded batch
      float v[8];
#pragma unroll
      for (int q = 0; q < 8; q++)
        if (r + q * 16 < f.rows) v[q] = f.part[(uint64_t)(r + q * 16) * f.k + c];
#pragma unroll
      for (int q = 0; q < 8; q++)
        if (r + q * 16 < f.rows) acc = combine(f.kind, acc, v[q]);
    }
  }
  part[ty][tx] = acc;
  __syncthreads();
  if (ty == 0 && c < f.k) {
    float v = part[0][tx];
#pragma unroll
    for (int l = 1; l < 16; l++) v = combine(f.kind, v, part[l][tx]);
    f.out[c] = v;
  }
}

void fold_jobs(hipStream_t s, const FoldJobs& jobs, uint32_t tiles) {
  if (jobs.n) hipLaunchKernelGGL(k_fold_jobs, dim3(tiles), dim3(1024), 0, s, jobs);
}

// Up to sixteen rows' loads in flight per thread (a K split has at most 16 partials, so one
// batch), added in row order (the order of k_split_sum). The last batch's loads are guarded
// rather than issued one by one, so a short fold waits for one memory latency, not one per row.
__global__ void __launch_bounds__(256) k_fold_wide(WideFolds jobs) {
  uint32_t j = 0;
  while (j + 1 < jobs.n && blockIdx.x >= jobs.job[j + 1].first_block) j++;
  const WideFold& f = jobs.job[j];
  const uint64_t i = ((uint64_t)(blockIdx.x - f.first_block) * 256 + threadIdx.x) * 4;
  if (i >= f.n) return;
  const float* p = f.part + i;
  float4 acc = *(const float4*)p;
  for (uint32_t r = 1; r < f.rows; r += 15) {
    float4 v[15];
#pragma unroll
    for (uint32_t q = 0; q < 15; q++)
      if (r + q < f.rows) v[q] = *(const float4*)(p + (uint64_t)(r + q) * f.n);
#pragma unroll
    for (uint32_t q = 0; q < 15; q++)
      if (r + q < f.rows) acc = make_float4(acc.x + v[q].x, acc.y + v[q].y, acc.z + v[q].z, acc.w + v[q].w);
  }
  *(float4*)(f.out + i) = acc;
}

void fold_wide(hipStream_t s, const WideFolds& jobs, uint32_t blocks) {
  if (jobs.n) hipLaunchKernelGGL(k_fold_wide, dim3(blocks), dim3(256), 0, s, jobs);
}

void fold_rows(hipStream_t s, int dtype, int kind, const void* partial, void* d, uint64_t rows, uint64_t k) {
  // The combining pass of reduce_cols: 16 row lanes per column, rows folded in order.
  dim3 g((uint32_t)blocks_for(k, 64), 1, 1);
  with_kind(kind, [&](auto K) {
    constexpr int KIND = decltype(K)::value;
    if (dtype == RG_F32)
      hipLaunchKernelGGL((k_reduce_cols<float, 16, KIND>), g, dim3(1024), 0, s, (const float*)partial, (float*)d, (uint32_t)rows, (uint32_t)k,
                         (uint32_t)rows, 1u);
    else
      hipLaunchKernelGGL((k_reduce_cols<double, 16, KIND>), g, dim3(1024), 0, s, (const double*)partial, (double*)d, (uint32_t)rows,
                         (uint32_t)k, (uint32_t)rows, 1u);
  });
}

void reduce_general(hipStream_t s, int dtype, int kind, const void* a, void* d, uint64_t out_n, const Strided& outer, const Strided& inner,
                    uint64_t red_n) {
  with_kind(kind, [&](auto K) {
    constexpr int KIND = decltype(K)::value;
    if (dtype == RG_F32) RG_LAUNCH((k_reduce_general<float, KIND>), out_n, (const float*)a, (float*)d, (uint32_t)out_n, outer, inner, (uint32_t)red_n);
    else RG_LAUNCH((k_reduce_general<double, KIND>), out_n, (const double*)a, (double*)d, (uint32_t)out_n, outer, inner, (uint32_t)red_n);
  });
}

__global__ void __launch_bounds__(TPB) k_copy_batch(CopyJobs jobs) {
  const int j = blockIdx.y;
  const uint64_t words = jobs.words[j];
  uint32_t* __restrict__ dst = jobs.dst[j];
  const uint32_t* __restrict__ src = jobs.src[j];
  const uint64_t first = (uint64_t)blockIdx.x * TPB + threadIdx.x, stride = (uint64_t)gridDim.x * TPB;
  if ((words & 3) == 0 && ((uintptr_t)dst & 15) == 0 && ((uintptr_t)src & 15) == 0) {  // 16 bytes per thread
    uint4* __restrict__ d4 = (uint4*)dst;
    const uint4* __restrict__ s4 = (const uint4*)src;
    for (uint64_t i = first; i < words / 4; i += stride) d4[i] = s4[i];
    return;
  }
  for (uint64_t i = first; i < words; i += stride) dst[i] = src[i];
}

__global__ void k_set_i32(int32_t* dst, int32_t value) { dst[0] = value; }

void copy_batch(hipStream_t s, const CopyJobs& jobs) {
  if (jobs.n <= 0) return;
  uint64_t most = 0;
  for (int j = 0; j < jobs.n; j++) most = std::max(most, jobs.words[j]);
  if (most == 0) return;
  const uint32_t bx = (uint32_t)std::min<uint64_t>((most + TPB - 1) / TPB, 1024);
  hipLaunchKernelGGL(k_copy_batch, dim3(bx, (uint32_t)jobs.n), dim3(TPB), 0, s, jobs);
}

void set_i32(hipStream_t s, int32_t* dst, int32_t value) { hipLaunchKernelGGL(k_set_i32, dim3(1), dim3(1), 0, s, dst, value); }

void copy_bytes(hipStream_t s, void* dst, const void* src, uint64_t bytes) {
  uint64_t words = bytes / 4;
  RG_LAUNCH(k_copy_words, words, (uint32_t*)dst, (const uint32_t*)src, words);
}

void record_history(hipStream_t s, int dtype, const void* slot, double* hist, const uint64_t* counter, uint64_t stride) {
  hipLaunchKernelGGL(k_record_history, dim3(1), dim3(1), 0, s, dtype, slot, hist, counter, stride);
}

void load_batch(hipStream_t s, void* dst, const void* batches, uint64_t bytes, uint64_t n_batches, const uint64_t* counter) {
  uint64_t words = bytes / 4;
  RG_LAUNCH(k_load_batch, words, (uint32_t*)dst, (const uint32_t*)batches, words, n_batches, counter);
}

void counter_inc(hipStream_t s, uint64_t* counter) { hipLaunchKernelGGL(k_counter_inc, dim3(1), dim3(1), 0, s, counter); }

void set_counter(hipStream_t s, uint64_t* counter, uint64_t value) { hipLaunchKernelGGL(k_set_counter, dim3(1), dim3(1), 0, s, counter, value); }

void hold_stream(hipStream_t s, double microseconds) {
  static uint64_t khz = [] {
    int dev = 0, rate = 0;
    hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&rate, hipDeviceAttributeWallClockRate, dev) != hipSuccess || rate <= 0) rate = 100000;
    return (uint64_t)rate;
  }();
  uint64_t ticks = (uint64_t)(microseconds * (double)khz / 1000.0);
  hipLaunchKernelGGL(k_hold, dim3(1), dim3(1), 0, s, ticks);
}

void fill_zero(hipStream_t s, void* dst, uint64_t bytes) {
  uint64_t words = bytes / 4;
  RG_LAUNCH(k_fill_zero, words, (uint32_t*)dst, words);
}

}  // namespace rgk
