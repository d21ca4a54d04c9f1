// Dense products for MatMul / MatMulT (reference src/plan.rs:1453-1493, flags from
// src/optimize.rs:338-350).
//
// fp32: a 128x128 block tile staged through LDS in K steps of 16, four wave64s each owning a
// 64x64 sub-tile computed with v_mfma_f32_32x32x2f32 (2x2 MFMA tiles, 64 accumulator registers
// per lane). Transposed operands are read through their flags: the loader transposes while
// staging, so no copy is made. Products whose output has too few tiles to fill 256 CUs split K
// and combine the partial sums in a fixed order (deterministic).
// fp64 and tiny or skinny fp32 products use a plain kernel, one thread per output element.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "kernels.h"

namespace rgk {

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 16, PAD = 4;
constexpr int LDA_S = BM + PAD, LDB_S = BN + PAD;

__device__ __forceinline__ int64_t batch_offset(const int64_t* offs, uint64_t stride, uint32_t b) {
  return offs ? offs[b] : (int64_t)(stride * b);
}

// Loads 8 consecutive elements of a row-major matrix row starting at column c, zero-filling
// past `cols` (and entirely when the row is out of range).
__device__ __forceinline__ void load8(const float* row, int64_t c, int64_t cols, bool row_ok, bool vec, float v[8]) {
  if (vec && row_ok && c + 8 <= cols) {
    float4 x = *(const float4*)(row + c);
    float4 y = *(const float4*)(row + c + 4);
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
    v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
  } else {
#pragma unroll
    for (int q = 0; q < 8; q++) v[q] = (row_ok && c + q < cols) ? row[c + q] : 0.0f;
  }
}

template <bool TA, bool TB>
__global__ void __launch_bounds__(256) k_gemm_mfma(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C,
                                                   int M, int N, int K, const int64_t* a_off, const int64_t* b_off, uint64_t a_stride,
                                                   uint64_t b_stride, int splits, int k_per_split, float* __restrict__ partial,
                                                   bool vec_a, bool vec_b) {
  __shared__ float As[2][BK][LDA_S];
  __shared__ float Bs[2][BK][LDB_S];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const uint32_t z = blockIdx.z;
  const uint32_t b = z / splits, sp = z % splits;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const float* Ab = A + batch_offset(a_off, a_stride, b);
  const float* Bb = B + batch_offset(b_off, b_stride, b);
  const int kbeg = sp * k_per_split, kend = min(K, kbeg + k_per_split);
  const int nk = (kend - kbeg + BK - 1) / BK;

  float ra[8], rb[8];
  // Thread roles in the loaders (256 threads x 8 elements = one 128x16 operand tile).
  auto load_tiles = [&](int k0) {
    if (!TA) {  // A is [M,K]: thread reads 8 consecutive k of row m
      int m = tid >> 1, kc = (tid & 1) * 8;
      load8(Ab + (int64_t)(m0 + m) * K, k0 + kc, kend, m0 + m < M, vec_a, ra);
    } else {    // A is [K,M]: thread reads 8 consecutive m of row k
      int k = tid >> 4, mc = (tid & 15) * 8;
      load8(Ab + (int64_t)(k0 + k) * M, m0 + mc, M, k0 + k < kend, vec_a, ra);
    }
    if (!TB) {  // B is [K,N]: 8 consecutive n of row k
      int k = tid >> 4, nc = (tid & 15) * 8;
      load8(Bb + (int64_t)(k0 + k) * N, n0 + nc, N, k0 + k < kend, vec_b, rb);
    } else {    // B is [N,K]: 8 consecutive k of row n
      int n = tid >> 1, kc = (tid & 1) * 8;
      load8(Bb + (int64_t)(n0 + n) * K, k0 + kc, kend, n0 + n < N, vec_b, rb);
    }
  };
  auto store_tiles = [&](int buf) {
    if (!TA) {
      int m = tid >> 1, kc = (tid & 1) * 8;
#pragma unroll
      for (int q = 0; q < 8; q++) As[buf][kc + q][m] = ra[q];
    } else {
      int k = tid >> 4, mc = (tid & 15) * 8;
      *(float4*)&As[buf][k][mc] = make_float4(ra[0], ra[1], ra[2], ra[3]);
      *(float4*)&As[buf][k][mc + 4] = make_float4(ra[4], ra[5], ra[6], ra[7]);
    }
    if (!TB) {
      int k = tid >> 4, nc = (tid & 15) * 8;
      *(float4*)&Bs[buf][k][nc] = make_float4(rb[0], rb[1], rb[2], rb[3]);
      *(float4*)&Bs[buf][k][nc + 4] = make_float4(rb[4], rb[5], rb[6], rb[7]);
    } else {
      int n = tid >> 1, kc = (tid & 1) * 8;
#pragma unroll
      for (int q = 0; q < 8; q++) Bs[buf][kc + q][n] = rb[q];
    }
  };

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
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
      float a0 = As[buf][kk + lk][wm * 64 + lrow];
      float a1 = As[buf][kk + lk][wm * 64 + 32 + lrow];
      float b0 = Bs[buf][kk + lk][wn * 64 + lrow];
      float b1 = Bs[buf][kk + lk][wn * 64 + 32 + lrow];
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
    }
    if (t + 1 < nk) store_tiles(buf ^ 1);
    __syncthreads();
  }
  // Accumulator register r of lane l holds row 8*(r/4) + 4*(l/32) + r%4, column l%32.
  float* out = splits > 1 ? partial + ((uint64_t)b * splits + sp) * (uint64_t)M * N : C + (uint64_t)b * M * N;
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
        int col = n0 + wn * 64 + j * 32 + lrow;
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

int split_count(uint64_t m, uint64_t n, uint64_t k, uint64_t batch) {
  uint64_t tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN) * batch;
  if (tiles >= 256 || k < 1024) return 1;
  uint64_t want = (512 + tiles - 1) / tiles;
  uint64_t most = k / 256;
  return (int)std::max<uint64_t>(1, std::min<uint64_t>(std::min(want, most), 32));
}

}  // namespace

uint64_t gemm_workspace(int dtype, uint64_t m, uint64_t n, uint64_t k, uint64_t batch) {
  if (!use_mfma(dtype, m, n, k)) return 0;
  int s = split_count(m, n, k, batch);
  return s > 1 ? (uint64_t)s * batch * m * n * sizeof(float) : 0;
}

void gemm(hipStream_t s, const GemmArgs& g) {
  if (g.m == 0 || g.n == 0 || g.batch == 0) return;
  if (use_mfma(g.dtype, g.m, g.n, g.k)) {
    int splits = split_count(g.m, g.n, g.k, g.batch);
    int kps = (int)(((g.k + splits - 1) / splits + BK - 1) / BK * BK);
    splits = (int)((g.k + kps - 1) / kps);
    auto aligned = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    bool offs_ok_a = g.a_off == nullptr && g.a_stride % 4 == 0;
    bool offs_ok_b = g.b_off == nullptr && g.b_stride % 4 == 0;
    // Vector loads run along K for A (untransposed) or M (transposed); likewise for B.
    bool vec_a = aligned(g.a) && offs_ok_a && ((g.ta ? g.m : g.k) % 4 == 0);
    bool vec_b = aligned(g.b) && offs_ok_b && ((g.tb ? g.k : g.n) % 4 == 0);
    dim3 grid((uint32_t)((g.n + BN - 1) / BN), (uint32_t)((g.m + BM - 1) / BM), (uint32_t)(g.batch * splits));
    float* part = splits > 1 ? (float*)g.workspace : nullptr;
    auto A = (const float*)g.a;
    auto B = (const float*)g.b;
    auto Cm = (float*)g.c;
    int M = (int)g.m, N = (int)g.n, K = (int)g.k;
#define RG_GEMM(TA, TB)                                                                                                     \
  hipLaunchKernelGGL((k_gemm_mfma<TA, TB>), grid, dim3(256), 0, s, A, B, Cm, M, N, K, g.a_off, g.b_off, g.a_stride, g.b_stride, \
                     splits, kps, part, vec_a, vec_b)
    if (!g.ta && !g.tb) RG_GEMM(false, false);
    else if (g.ta && !g.tb) RG_GEMM(true, false);
    else if (!g.ta && g.tb) RG_GEMM(false, true);
    else RG_GEMM(true, true);
#undef RG_GEMM
    if (splits > 1) {
      uint64_t mn = g.m * g.n;
      hipLaunchKernelGGL(k_split_sum, dim3((uint32_t)((mn + 255) / 256), (uint32_t)g.batch), dim3(256), 0, s, (const float*)part, Cm, mn, splits);
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
