// Dense products for MatMul / MatMulT (reference src/plan.rs:1453-1493, flags from
// src/optimize.rs:338-350).
//
// fp32: block tiles of 128x128, 128x64, 64x128, 64x64, 128x32 or 32x128 staged through LDS in
// K steps of 16, four wave64s per block each owning 32x32 MFMA tiles (v_mfma_f32_32x32x2f32).
// Transposed operands are read through their flags: the loader transposes while staging, so no
// copy is made. The tile is chosen per product so that the launch fills 256 CUs with little
// padding (32-wide tiles for 32-wide attention heads); products whose output still has too few
// tiles split K and combine the partial sums in a fixed order (deterministic).
// fp64 and tiny or skinny fp32 products use a plain kernel, one thread per output element.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "kernels.h"

namespace rgk {

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int PAD = 4;

__device__ __forceinline__ int64_t batch_offset(const int64_t* offs, uint64_t stride, uint32_t b) {
  return offs ? offs[b] : (int64_t)(stride * b);
}

// Loads N (2, 4 or 8) consecutive elements of a row-major row starting at column c, zero-filling
// past `cols` and when the row is out of range. `vec`: the row and c allow 16/8-byte loads.
template <int N>
__device__ __forceinline__ void loadn(const float* row, int64_t c, int64_t cols, bool row_ok, bool vec, float v[N]) {
  if (vec && row_ok && c + N <= cols) {
    if constexpr (N == 2) {
      float2 x = *(const float2*)(row + c);
      v[0] = x.x; v[1] = x.y;
    } else {
#pragma unroll
      for (int q = 0; q < N; q += 4) {
        float4 x = *(const float4*)(row + c + q);
        v[q] = x.x; v[q + 1] = x.y; v[q + 2] = x.z; v[q + 3] = x.w;
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < N; q++) v[q] = (row_ok && c + q < cols) ? row[c + q] : 0.0f;
  }
}

// Which output tile a block computes. The dispatcher deals consecutive blocks round-robin over
// the 8 XCDs, each with its own L2; with `swizzle`, XCD x instead receives the contiguous run
// x*nb/8 ... (x+1)*nb/8 - 1 of tiles, and within a batch the tiles run in groups of 8 M-panels
// per N sweep, so blocks resident on one XCD share their A and B panels in its L2.
struct TileIndex {
  uint32_t tm, tn, z;
};

__device__ __forceinline__ TileIndex tile_of(uint32_t tiles_m, uint32_t tiles_n, int swizzle) {
  uint32_t nb = gridDim.x, bid = blockIdx.x;
  uint32_t per_batch = tiles_m * tiles_n;
  if (!swizzle) return {(bid % per_batch) / tiles_n, bid % tiles_n, bid / per_batch};
  uint32_t lid = (nb % 8 == 0) ? (bid % 8) * (nb / 8) + bid / 8 : bid;
  uint32_t z = lid / per_batch, t = lid % per_batch;
  constexpr uint32_t GROUP = 8;
  uint32_t span = GROUP * tiles_n;
  uint32_t first = (t / span) * GROUP;
  uint32_t rows = min(tiles_m - first, GROUP);
  uint32_t in = t % span;
  return {first + in % rows, in / rows, z};
}

// C = op(A) op(B) for one BM x BN block tile. Four wave64s in a WM x WN grid; each wave owns a
// (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA tiles (v_mfma_f32_32x32x2f32). Operands are staged
// through double-buffered LDS in K steps of BK, K-major, so each MFMA operand is one
// conflict-free 32-lane LDS row read; transposed operands are transposed while staging.
// The grid is one-dimensional: tiles_m * tiles_n * batch * splits blocks (tile_of).
template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB>
__global__ void __launch_bounds__(256) k_gemm_mfma(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C,
                                                   int M, int N, int K, const int64_t* a_off, const int64_t* b_off, uint64_t a_stride,
                                                   uint64_t b_stride, int splits, int k_per_split, float* __restrict__ partial,
                                                   bool vec_a, bool vec_b, uint32_t tiles_m, uint32_t tiles_n, int swizzle) {
  static_assert(WM * WN == 4, "four waves");
  constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
  static_assert(TM >= 1 && TN >= 1, "wave tile of at least 32x32");
  // Loader geometry: 256 threads cover a BM x BK (A) and a BK x BN (B) tile.
  constexpr int EA = BM * BK / 256, EB = BN * BK / 256;
  __shared__ float As[2][BK][BM + PAD];
  __shared__ float Bs[2][BK][BN + PAD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const TileIndex ti = tile_of(tiles_m, tiles_n, swizzle);
  const uint32_t b = ti.z / splits, sp = ti.z % splits;
  const int m0 = ti.tm * BM, n0 = ti.tn * BN;
  const float* Ab = A + batch_offset(a_off, a_stride, b);
  const float* Bb = B + batch_offset(b_off, b_stride, b);
  const int kbeg = sp * k_per_split, kend = min(K, kbeg + k_per_split);
  const int nk = (kend - kbeg + BK - 1) / BK;

  float ra[EA], rb[EB];
  auto load_tiles = [&](int k0) {
    if (!TA) {  // A is [M,K]: BM rows of BK k
      constexpr int TPR = BK / EA;
      int m = tid / TPR, kc = (tid % TPR) * EA;
      loadn<EA>(Ab + (int64_t)(m0 + m) * K, k0 + kc, kend, m0 + m < M, vec_a, ra);
    } else {    // A is [K,M]: BK rows of BM m
      constexpr int TPR = BM / EA;
      int k = tid / TPR, mc = (tid % TPR) * EA;
      loadn<EA>(Ab + (int64_t)(k0 + k) * M, m0 + mc, M, k0 + k < kend, vec_a, ra);
    }
    if (!TB) {  // B is [K,N]: BK rows of BN n
      constexpr int TPR = BN / EB;
      int k = tid / TPR, nc = (tid % TPR) * EB;
      loadn<EB>(Bb + (int64_t)(k0 + k) * N, n0 + nc, N, k0 + k < kend, vec_b, rb);
    } else {    // B is [N,K]: BN rows of BK k
      constexpr int TPR = BK / EB;
      int n = tid / TPR, kc = (tid % TPR) * EB;
      loadn<EB>(Bb + (int64_t)(n0 + n) * K, k0 + kc, kend, n0 + n < N, vec_b, rb);
    }
  };
  auto store_tiles = [&](int buf) {
    if (!TA) {
      constexpr int TPR = BK / EA;
      int m = tid / TPR, kc = (tid % TPR) * EA;
#pragma unroll
      for (int q = 0; q < EA; q++) As[buf][kc + q][m] = ra[q];
    } else {
      constexpr int TPR = BM / EA;
      int k = tid / TPR, mc = (tid % TPR) * EA;
#pragma unroll
      for (int q = 0; q < EA; q++) As[buf][k][mc + q] = ra[q];
    }
    if (!TB) {
      constexpr int TPR = BN / EB;
      int k = tid / TPR, nc = (tid % TPR) * EB;
#pragma unroll
      for (int q = 0; q < EB; q++) Bs[buf][k][nc + q] = rb[q];
    } else {
      constexpr int TPR = BK / EB;
      int n = tid / TPR, kc = (tid % TPR) * EB;
#pragma unroll
      for (int q = 0; q < EB; q++) Bs[buf][kc + q][n] = rb[q];
    }
  };

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

  if (nk > 0) {
    load_tiles(kbeg);
    store_tiles(0);
  }
  __syncthreads();
  const int lrow = lane & 31, lk = lane >> 5;
  for (int t = 0; t < nk; t++) {
    const int buf = t & 1;
    if (t + 1 < nk) load_tiles(kbeg + (t + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 2) {
      float av[TM], bv[TN];
#pragma unroll
      for (int i = 0; i < TM; i++) av[i] = As[buf][kk + lk][wm * WTM + i * 32 + lrow];
#pragma unroll
      for (int j = 0; j < TN; j++) bv[j] = Bs[buf][kk + lk][wn * WTN + j * 32 + lrow];
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (t + 1 < nk) store_tiles(buf ^ 1);
    __syncthreads();
  }
  // Accumulator register r of lane l holds row 8*(r/4) + 4*(l/32) + r%4, column l%32.
  float* out = splits > 1 ? partial + ((uint64_t)b * splits + sp) * (uint64_t)M * N : C + (uint64_t)b * M * N;
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        int row = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
        int col = n0 + wn * WTN + j * 32 + lrow;
        if (row < M && col < N) out[(uint64_t)row * N + col] = acc[i][j][r];
      }
}

__global__ void __launch_bounds__(256) k_split_sum(const float* __restrict__ partial, float* __restrict__ C, uint64_t mn, int splits) {
  uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  uint32_t b = blockIdx.y;
  if (i >= mn) return;
  float acc = partial[((uint64_t)b * splits) * mn + i];
  for (int s = 1; s < splits; s++) acc += partial[((uint64_t)b * splits + s) * mn + i];
  C[(uint64_t)b * mn + i] = acc;
}

// One output element per thread; k ascending.
template <class T>
__global__ void __launch_bounds__(256) k_gemm_plain(const T* __restrict__ A, const T* __restrict__ B, T* __restrict__ C, uint32_t M,
                                                    uint32_t N, uint32_t K, bool ta, bool tb, const int64_t* a_off, const int64_t* b_off,
                                                    uint64_t a_stride, uint64_t b_stride) {
  uint32_t b = blockIdx.y;
  uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (uint64_t)M * N) return;
  uint32_t i = (uint32_t)(t / N), j = (uint32_t)(t % N);
  const T* a = A + batch_offset(a_off, a_stride, b);
  const T* bb = B + batch_offset(b_off, b_stride, b);
  T acc = (T)0;
  for (uint32_t p = 0; p < K; p++) {
    T x = ta ? a[(uint64_t)p * M + i] : a[(uint64_t)i * K + p];
    T y = tb ? bb[(uint64_t)j * K + p] : bb[(uint64_t)p * N + j];
    acc = acc + x * y;
  }
  C[(uint64_t)b * M * N + t] = acc;
}

bool use_mfma(int dtype, uint64_t m, uint64_t n, uint64_t k) {
  return dtype == RG_F32 && m >= 32 && n >= 32 && k >= 8 && m * n * k >= (1u << 18);
}

struct TileCfg {
  int bm, bn, bk;
};

// Block tile, from measurements of C4's products on MI355X (K steps of 32 hide more load latency
// for the smaller tiles): 32-wide tiles for outputs 32..96 wide or 32 tall (attention heads,
// the vocabulary), the largest square-ish tile that still yields two blocks per CU (512), else
// 64x64 (split over K later when even that leaves the CUs idle).
TileCfg pick_tile(uint64_t m, uint64_t n, uint64_t batch) {
  auto blocks = [&](int bm, int bn) { return ((m + bm - 1) / bm) * ((n + bn - 1) / bn) * batch; };
  if (n <= 96 && n % 32 == 0) return {128, 32, 32};
  if (m <= 32) return {32, 128, 32};
  if (blocks(128, 128) >= 512) return {128, 128, 16};
  if (blocks(128, 64) >= 512) return {128, 64, 32};
  return {64, 64, 32};
}

int split_count(const TileCfg& t, uint64_t m, uint64_t n, uint64_t k, uint64_t batch) {
  uint64_t tiles = ((m + t.bm - 1) / t.bm) * ((n + t.bn - 1) / t.bn) * batch;
  if (tiles >= 256 || k < 1024) return 1;
  uint64_t want = (512 + tiles - 1) / tiles;
  uint64_t most = k / 512;
  return (int)std::max<uint64_t>(1, std::min<uint64_t>(std::min(want, most), 16));
}

template <int BM, int BN, int BK, int WM, int WN>
void launch_flags(hipStream_t s, bool ta, bool tb, dim3 grid, const float* A, const float* B, float* C, int M, int N, int K,
                  const int64_t* a_off, const int64_t* b_off, uint64_t as, uint64_t bs, int splits, int kps, float* part, bool va,
                  bool vb, uint32_t tm, uint32_t tn, int swizzle) {
#define RG_GEMM(TA_, TB_)                                                                                                     \
  hipLaunchKernelGGL((k_gemm_mfma<BM, BN, BK, WM, WN, TA_, TB_>), grid, dim3(256), 0, s, A, B, C, M, N, K, a_off, b_off, as, bs, \
                     splits, kps, part, va, vb, tm, tn, swizzle)
  if (!ta && !tb) RG_GEMM(false, false);
  else if (ta && !tb) RG_GEMM(true, false);
  else if (!ta && tb) RG_GEMM(false, true);
  else RG_GEMM(true, true);
#undef RG_GEMM
}

// Instantiates the tile shapes pick_tile can return.
void launch_mfma(hipStream_t s, const TileCfg& t, bool ta, bool tb, dim3 grid, const float* A, const float* B, float* C, int M, int N,
                 int K, const int64_t* a_off, const int64_t* b_off, uint64_t as, uint64_t bs, int splits, int kps, float* part, bool va,
                 bool vb, uint32_t tm, uint32_t tn, int swizzle) {
#define RG_TILE(BM_, BN_, BK_, WM_, WN_)                                                                                      \
  if (t.bm == BM_ && t.bn == BN_ && t.bk == BK_)                                                                               \
    return launch_flags<BM_, BN_, BK_, WM_, WN_>(s, ta, tb, grid, A, B, C, M, N, K, a_off, b_off, as, bs, splits, kps, part, va, vb, \
                                                 tm, tn, swizzle)
  RG_TILE(128, 128, 16, 2, 2);
  RG_TILE(128, 64, 16, 2, 2);
  RG_TILE(64, 128, 16, 2, 2);
  RG_TILE(64, 64, 16, 2, 2);
  RG_TILE(128, 32, 16, 4, 1);
  RG_TILE(32, 128, 16, 1, 4);
  RG_TILE(128, 128, 32, 2, 2);
  RG_TILE(128, 64, 32, 2, 2);
  RG_TILE(64, 128, 32, 2, 2);
  RG_TILE(64, 64, 32, 2, 2);
  RG_TILE(128, 32, 32, 4, 1);
  RG_TILE(32, 128, 32, 1, 4);
#undef RG_TILE
}

}  // namespace

uint64_t gemm_workspace(int dtype, uint64_t m, uint64_t n, uint64_t k, uint64_t batch) {
  if (!use_mfma(dtype, m, n, k)) return 0;
  int s = split_count(pick_tile(m, n, batch), m, n, k, batch);
  return s > 1 ? (uint64_t)s * batch * m * n * sizeof(float) : 0;
}

void gemm(hipStream_t s, const GemmArgs& g) {
  if (g.m == 0 || g.n == 0 || g.batch == 0) return;
  if (use_mfma(g.dtype, g.m, g.n, g.k)) {
    TileCfg t = pick_tile(g.m, g.n, g.batch);
    int splits = split_count(t, g.m, g.n, g.k, g.batch);
    int kps = (int)(((g.k + splits - 1) / splits + t.bk - 1) / t.bk * t.bk);
    splits = (int)((g.k + kps - 1) / kps);
    auto aligned = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    bool offs_ok_a = g.a_off == nullptr && g.a_stride % 4 == 0;
    bool offs_ok_b = g.b_off == nullptr && g.b_stride % 4 == 0;
    // Vector loads run along K for A (untransposed) or M (transposed); likewise for B.
    bool vec_a = aligned(g.a) && offs_ok_a && ((g.ta ? g.m : g.k) % 4 == 0);
    bool vec_b = aligned(g.b) && offs_ok_b && ((g.tb ? g.k : g.n) % 4 == 0);
    uint32_t tiles_m = (uint32_t)((g.m + t.bm - 1) / t.bm), tiles_n = (uint32_t)((g.n + t.bn - 1) / t.bn);
    dim3 grid((uint32_t)(tiles_m * tiles_n * g.batch * splits));
    float* part = splits > 1 ? (float*)g.workspace : nullptr;
    launch_mfma(s, t, g.ta, g.tb, grid, (const float*)g.a, (const float*)g.b, (float*)g.c, (int)g.m, (int)g.n, (int)g.k, g.a_off,
                g.b_off, g.a_stride, g.b_stride, splits, kps, part, vec_a, vec_b, tiles_m, tiles_n, 1);
    if (splits > 1) {
      uint64_t mn = g.m * g.n;
      hipLaunchKernelGGL(k_split_sum, dim3((uint32_t)((mn + 255) / 256), (uint32_t)g.batch), dim3(256), 0, s, (const float*)part,
                         (float*)g.c, mn, splits);
    }
    return;
  }
  dim3 grid((uint32_t)((g.m * g.n + 255) / 256), (uint32_t)g.batch);
  if (g.dtype == RG_F32)
    hipLaunchKernelGGL(k_gemm_plain<float>, grid, dim3(256), 0, s, (const float*)g.a, (const float*)g.b, (float*)g.c, (uint32_t)g.m,
                       (uint32_t)g.n, (uint32_t)g.k, g.ta, g.tb, g.a_off, g.b_off, g.a_stride, g.b_stride);
  else
    hipLaunchKernelGGL(k_gemm_plain<double>, grid, dim3(256), 0, s, (const double*)g.a, (const double*)g.b, (double*)g.c, (uint32_t)g.m,
                       (uint32_t)g.n, (uint32_t)g.k, g.ta, g.tb, g.a_off, g.b_off, g.a_stride, g.b_stride);
}

}  // namespace rgk
