// Dense products for MatMul / MatMulT (reference src/plan.rs:1453-1493, flags from
// src/optimize.rs:338-350).
//
// fp32: block tiles from 128x128 down to 128x32 / 32x128, four or eight wave64s per block, each
// wave owning a grid of 16x16 MFMA tiles (v_mfma_f32_16x16x4f32), or of 32x32 ones
// (v_mfma_f32_32x32x2f32) for some shapes. Global loads run two K steps ahead through two register
// stages, and operands are staged through double-buffered LDS in their own global layout, so no
// operand is transposed while staging:
//  - a K-contiguous operand (A, or B when transposed) sits in LDS as [rows][BK + 4]; one 16-byte
//    LDS read gives a lane four consecutive k of one tile row, feeding four MFMA k-steps;
//  - an M- or N-contiguous operand sits as [BK][cols]; one read gives a lane T consecutive
//    columns at one k, one for each of the wave's T tiles (tile t holds columns t, t + T, ...).
// Global loads are 16-byte vectors without branches: a vector lies wholly inside or outside the
// operand (leading dimensions are multiples of 4), and an outside vector reads a valid address
// and is replaced by zeros; products whose tiles divide M, N and K skip even that check. The tile
// is chosen per product to fill 256 CUs with little padding (32-wide tiles for 32-wide attention
// heads); products whose output still has too few tiles split K and combine the partial sums in a
// fixed order (deterministic). Unaligned operands take the same kernel with scalar loads.
// fp32 products with at most 16 rows and a long K, or a K of at most 16, stream through the
// skinny kernels below (HBM-bound shapes); fp64 and the remaining tiny products use a plain
// kernel, one thread per output element.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <stdexcept>
#include <string>

#include "gemm_mfma.h"
#include "kernels.h"
#include "ops.h"

namespace rgk {

namespace {

using namespace rgg;

template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, int MODE, int MS>
__global__ void __launch_bounds__(64 * WM * WN) k_gemm_mfma(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C,
                                                           int M, int N, int K, const int64_t* a_off, const int64_t* b_off,
                                                           uint64_t a_stride, uint64_t b_stride, int splits, int k_per_split,
                                                           float* __restrict__ partial, const float* __restrict__ bias, uint32_t tiles_m,
                                                           uint32_t tiles_n, int swizzle) {
  rgg::StoreC epi{C, partial, splits, (uint64_t)M * N};
  rgg::gemm_mfma_block<BM, BN, BK, WM, WN, TA, TB, MODE, MS>(A, B, M, N, K, a_off, b_off, a_stride, b_stride, splits, k_per_split, bias,
                                                              tiles_m, tiles_n, swizzle, epi);
}

// One unbatched product's share of a grouped launch (k_gemm_mfma_group).
struct GroupPart {
  const float *a, *b;
  float *c, *part;
  const float* bias;
  int m, n, k, splits, kps;
  uint32_t tm, tn, blocks;
};
constexpr int GROUP_MAX = 3;
struct GroupParts {
  GroupPart p[GROUP_MAX];
};

// Part I of a grouped launch: flags bits 2I (TB) and 2I + 1 (TA).
template <int BM, int BN, int BK, int WM, int WN, int FLAGS, int I>
__device__ __forceinline__ void group_part(const GroupPart& p, uint32_t bid, float* smem) {
  constexpr bool TA = (FLAGS >> (2 * I + 1)) & 1, TB = (FLAGS >> (2 * I)) & 1;
  StoreC epi{p.c, p.part, p.splits, (uint64_t)p.m * p.n};
  gemm_mfma_tile<BM, BN, BK, WM, WN, TA, TB, LOAD_EVEN, 16>(p.a, p.b, p.m, p.n, p.k, nullptr, nullptr, 0, 0, p.splits, p.kps, p.bias, p.tm,
                                                             p.tn, 1, epi, bid, p.blocks, smem);
}

template <int BM, int BN, int BK, int FLAGS, int I>
constexpr int part_lds() {
  return TileLds<BM, BN, BK, ((FLAGS >> (2 * I + 1)) & 1) != 0, ((FLAGS >> (2 * I)) & 1) != 0>::FLOATS;
}

// N independent unbatched products on one tile shape in one launch: part i takes the next
// p[i].blocks blocks, all staging through the same LDS. Each block runs the code of a single
// product's launch, so every output gets the same bits; the launch's fixed cost is paid once,
// and the parts' grids (each about one block per CU) run side by side.
template <int BM, int BN, int BK, int WM, int WN, int N, int FLAGS>
__global__ void __launch_bounds__(64 * WM * WN) k_gemm_mfma_group(GroupParts g) {
  constexpr int F0 = part_lds<BM, BN, BK, FLAGS, 0>(), F1 = part_lds<BM, BN, BK, FLAGS, 1>();
  constexpr int F2 = N > 2 ? part_lds<BM, BN, BK, FLAGS, 2>() : 0;
  constexpr int F01 = F0 > F1 ? F0 : F1;
  __shared__ float smem[F01 > F2 ? F01 : F2];
  uint32_t bid = blockIdx.x;
  if (bid < g.p[0].blocks) return group_part<BM, BN, BK, WM, WN, FLAGS, 0>(g.p[0], bid, smem);
  bid -= g.p[0].blocks;
  if (N == 2 || bid < g.p[1].blocks) return group_part<BM, BN, BK, WM, WN, FLAGS, 1>(g.p[1], bid, smem);
  if constexpr (N > 2) group_part<BM, BN, BK, WM, WN, FLAGS, 2>(g.p[2], bid - g.p[1].blocks, smem);
}

// Sums the K-split partial products in split order. Four outputs per thread (16-byte loads when
// M N is a multiple of 4), all splits' loads issued before the adds.
__global__ void __launch_bounds__(256) k_split_sum(const float* __restrict__ partial, float* __restrict__ C, uint64_t mn, int splits,
                                                   const float* __restrict__ bias, uint64_t n) {
  const uint64_t i = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  const uint32_t b = blockIdx.y;
  if (i >= mn) return;
  const float* p = partial + (uint64_t)b * splits * mn + i;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (mn % 4 == 0) {
    float4 v[16];
#pragma unroll
    for (int s = 0; s < 16; s++)
      if (s < splits) v[s] = *(const float4*)(p + (uint64_t)s * mn);
    acc = v[0];
#pragma unroll
    for (int s = 1; s < 16; s++)
      if (s < splits) acc = make_float4(acc.x + v[s].x, acc.y + v[s].y, acc.z + v[s].z, acc.w + v[s].w);
    if (bias) acc = make_float4(acc.x + bias[i % n], acc.y + bias[(i + 1) % n], acc.z + bias[(i + 2) % n], acc.w + bias[(i + 3) % n]);
    *(float4*)(C + (uint64_t)b * mn + i) = acc;
    return;
  }
  for (uint64_t e = i; e < i + 4 && e < mn; e++) {
    float x = partial[(uint64_t)b * splits * mn + e];
    for (int s = 1; s < splits; s++) x += partial[((uint64_t)b * splits + s) * mn + e];
    if (bias) x += bias[e % n];
    C[(uint64_t)b * mn + e] = x;
  }
}

// C[e] += bias[e mod n]: the bias of a product that does not run on the matrix cores.
__global__ void __launch_bounds__(256) k_add_bias(float* __restrict__ C, const float* __restrict__ bias, uint64_t total, uint64_t n) {
  const uint64_t e = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (e < total) C[e] = C[e] + bias[e % n];
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

// ---- skinny fp32 products: HBM-bound shapes streamed at full bandwidth -------------------------
//
// Products with at most 16 rows and a long K (a few vectors against a large matrix), or with a
// K of at most 16 (outer products), do about 4 flops per byte they move: the matrix cores cannot
// speed them up, the number of bytes in flight can. Each kernel reads its large operand exactly
// once with 16-byte loads and fixes the order of every sum, so results are deterministic.

// C (M <= MR rows) = op(A) B with B row-major K x N (N % 4 == 0, 16-byte aligned). A block of
// four waves owns 256 columns (a float4 per lane) and one K split; its waves take consecutive
// quarters of the split, sum their k in increasing order, and combine in wave order through
// LDS. With several splits, split s writes partials [s][M N], summed in split order afterwards.
// The loop has no branches: a wave's K range is made uniform (readfirstlane), so op(A) values are
// scalar loads that never wait on the B rows in flight; rows m >= M read row M - 1 and columns
// past N read the last column, and neither is stored.
template <int MR>
struct RowsLds {
  static constexpr int FLOAT4S = 3 * MR * 64;  // the sums of waves 1..3; wave 0 keeps its own
};

// op(A) of the streaming kernels, read through the constant address space: the launch never
// writes it, and so its wave-uniform loads are scalar loads also where the block code runs inside
// a grouped launch, whose operand pointers come from a struct and carry no __restrict__.
typedef const __attribute__((address_space(4))) float* ConstOperand;

// Block (bx, by) of k_gemm_skinny_rows, its wave sums combined through `lds`.
template <int MR, int UNROLL = 8>
__device__ __forceinline__ void skinny_rows_block(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ out, int M,
                                                  int N, int K, bool ta, int kps, uint32_t bx, uint32_t by, float4* lds) {
  float4(*red)[MR][64] = (float4(*)[MR][64])lds;
  const ConstOperand Ac = (ConstOperand)A;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int col = (bx * 64 + lane) * 4;
  const int colr = min(col, N - 4);
  const int k0 = by * kps, k1 = min(K, k0 + kps);
  const int quarter = (k1 - k0 + 3) / 4;
  const int kw0 = min(k1, k0 + wave * quarter), kw1 = min(k1, kw0 + quarter);
  const uint64_t sm = ta ? 1 : (uint64_t)K, sk = ta ? (uint64_t)M : 1;  // op(A)[m][k] = A[m * sm + k * sk]
  float4 acc[MR];
#pragma unroll
  for (int m = 0; m < MR; m++) acc[m] = make_float4(0.f, 0.f, 0.f, 0.f);
  int k = kw0;
  for (; k + UNROLL <= kw1; k += UNROLL) {
    float4 b[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; u++) b[u] = *(const float4*)(B + (uint64_t)(k + u) * N + colr);
#pragma unroll
    for (int u = 0; u < UNROLL; u++)
#pragma unroll
      for (int m = 0; m < MR; m++) {
        const float a = Ac[(uint64_t)min(m, M - 1) * sm + (uint64_t)(k + u) * sk];
        acc[m] = make_float4(fmaf(a, b[u].x, acc[m].x), fmaf(a, b[u].y, acc[m].y), fmaf(a, b[u].z, acc[m].z), fmaf(a, b[u].w, acc[m].w));
      }
  }
  for (; k < kw1; k++) {
    const float4 b = *(const float4*)(B + (uint64_t)k * N + colr);
#pragma unroll
    for (int m = 0; m < MR; m++) {
      const float a = Ac[(uint64_t)min(m, M - 1) * sm + (uint64_t)k * sk];
      acc[m] = make_float4(fmaf(a, b.x, acc[m].x), fmaf(a, b.y, acc[m].y), fmaf(a, b.z, acc[m].z), fmaf(a, b.w, acc[m].w));
    }
  }
  if (wave > 0)
#pragma unroll
    for (int m = 0; m < MR; m++) red[wave - 1][m][lane] = acc[m];
  __syncthreads();
  if (wave != 0 || col >= N) return;
  float* dst = out + (uint64_t)by * M * N;
#pragma unroll
  for (int m = 0; m < MR; m++)
    if (m < M) {
      float4 v = acc[m];
#pragma unroll
      for (int w = 0; w < 3; w++) {
        const float4 x = red[w][m][lane];
        v = make_float4(v.x + x.x, v.y + x.y, v.z + x.z, v.w + x.w);
      }
      *(float4*)(dst + (uint64_t)m * N + col) = v;
    }
}

// C (M <= MR rows) = A B^T with A row-major M x K and B stored N x K (N % NC == 0, K % 256 == 0,
// both 16-byte aligned): every output is the dot product of two contiguous rows. A block owns
// 4 NC consecutive columns of C (NC per wave) and one K split of `kps` (a multiple of 256, at
// most DOT_KPS); it copies its A panel to LDS while its first B rows load, so the loop's only
// global loads are the B rows, four float4 steps deep. Lanes take k in float4 steps 256 apart, each lane summing its
// share in increasing k; the 64 lane sums combine by a fixed xor butterfly, and with several
// splits, split s writes partials [s][M N], summed in split order afterwards. Rows m >= M read
// row M - 1 and are not stored. (For 16 rows the split is at most DOT_KPS / 2.)
constexpr int DOT_KPS = 1024;
template <int MR>
struct DotLds {
  static constexpr int KPS_MAX = MR <= 8 ? DOT_KPS : DOT_KPS / 2;  // a 32 KiB panel either way
  static constexpr int FLOAT4S = MR * KPS_MAX / 4;
};

// Block (bx, by) of a k_gemm_skinny_dot grid of ny splits, its A panel in `lds`.
template <int MR, int NC>
__device__ __forceinline__ void skinny_dot_block(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ out, int M,
                                                 int N, int K, int kps, uint32_t bx, uint32_t by, uint32_t ny, float4* lds) {
  constexpr int KPS_MAX = DotLds<MR>::KPS_MAX;
  float4(*panel)[KPS_MAX / 4] = (float4(*)[KPS_MAX / 4])lds;
  const int lane = threadIdx.x & 63;
  // Blocks side by side take different K chunks (rotated by the column tile), so concurrent
  // blocks read B at addresses spread over the rows rather than one column range of every row.
  const int split = (by + bx) % ny;
  const int k0 = split * kps, len = min(K - k0, kps);
  const int n0 = (bx * 4 + (threadIdx.x >> 6)) * NC;
  const bool active = n0 < N;
  const int nr = active ? n0 : N - NC;  // an idle wave reads valid rows and stores nothing
  // The first four steps of B rows are issued before the panel copy, so their latency overlaps it.
  auto load = [&](float4 (&b)[4][NC], int kk) {
#pragma unroll
    for (int h = 0; h < 4; h++)
#pragma unroll
      for (int c = 0; c < NC; c++)
        b[h][c] = kk + h * 256 < len ? *(const float4*)(B + (uint64_t)(nr + c) * K + k0 + kk + h * 256) : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  float4 b[4][NC];
  load(b, lane * 4);
  for (int q = threadIdx.x; q < MR * (len / 4); q += 256) {
    const int m = q / (len / 4), c = q % (len / 4);
    panel[m][c] = *(const float4*)(A + (uint64_t)min(m, M - 1) * K + k0 + 4 * c);
  }
  __syncthreads();
  if (!active) return;
  float acc[MR][NC];
#pragma unroll
  for (int m = 0; m < MR; m++)
#pragma unroll
    for (int c = 0; c < NC; c++) acc[m][c] = 0.f;
  for (int kk = lane * 4; kk < len; kk += 1024) {
#pragma unroll
    for (int h = 0; h < 4; h++)
      if (kk + h * 256 < len)
#pragma unroll
        for (int m = 0; m < MR; m++) {
          const float4 a = panel[m][(kk + h * 256) / 4];
#pragma unroll
          for (int c = 0; c < NC; c++)
            acc[m][c] = fmaf(a.w, b[h][c].w, fmaf(a.z, b[h][c].z, fmaf(a.y, b[h][c].y, fmaf(a.x, b[h][c].x, acc[m][c]))));
        }
    if (kk + 1024 < len) load(b, kk + 1024);
  }
  float* dst = out + (uint64_t)split * M * N;
#pragma unroll
  for (int m = 0; m < MR; m++)
#pragma unroll
    for (int c = 0; c < NC; c++) {
      const float v = rg_wave_sum(acc[m][c]);
      if (m < M && lane == 0) dst[(uint64_t)m * N + n0 + c] = v;
    }
}

// C (M x N, N % 4 == 0) = op(A) op(B) with K <= KR (an outer product of a few vectors): write
// bound. A block of four waves owns 256 columns; each lane keeps its float4 of every op(B) row in
// registers and walks the wave's rows, reading op(A)'s row values as wave-uniform scalars. The
// output is written with non-temporal stores: it is large (a full matrix from a few vectors) and
// streaming it past the caches leaves them to the operands of the kernels that follow (4 % off a
// C5 pass on MI355X).
// Block (bx, by) of k_gemm_outer.
template <int KR, bool TA, bool TB>
__device__ __forceinline__ void outer_block(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N,
                                            int K, int rows_per_wave, uint32_t bx, uint32_t by) {
  const ConstOperand Ac = (ConstOperand)A;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int col = (bx * 64 + lane) * 4;
  if (col >= N) return;
  // Rows k >= K are zeros: the extra terms add exact zeros, so the sums are unchanged.
  float4 b[KR];
#pragma unroll
  for (int k = 0; k < KR; k++) {
    if (k < K) {
      if (TB) b[k] = make_float4(B[(uint64_t)col * K + k], B[(uint64_t)(col + 1) * K + k], B[(uint64_t)(col + 2) * K + k], B[(uint64_t)(col + 3) * K + k]);
      else b[k] = *(const float4*)(B + (uint64_t)k * N + col);
    } else {
      b[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  const int r0 = (by * 4 + wave) * rows_per_wave, r1 = min(M, r0 + rows_per_wave);
  for (int i = r0; i < r1; i++) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < KR; k++) {
      const float a = k < K ? (TA ? Ac[(uint64_t)k * M + i] : Ac[(uint64_t)i * K + k]) : 0.f;
      acc = make_float4(fmaf(a, b[k].x, acc.x), fmaf(a, b[k].y, acc.y), fmaf(a, b[k].z, acc.z), fmaf(a, b[k].w, acc.w));
    }
    __builtin_nontemporal_store(floatx4{acc.x, acc.y, acc.z, acc.w}, (floatx4*)(C + (uint64_t)i * N + col));
  }
}

template <int MR, int UNROLL = 8>
__global__ void __launch_bounds__(256) k_gemm_skinny_rows(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ out,
                                                          int M, int N, int K, bool ta, int kps) {
  __shared__ float4 lds[RowsLds<MR>::FLOAT4S];
  skinny_rows_block<MR, UNROLL>(A, B, out, M, N, K, ta, kps, blockIdx.x, blockIdx.y, lds);
}

template <int MR, int NC>
__global__ void __launch_bounds__(256) k_gemm_skinny_dot(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ out,
                                                         int M, int N, int K, int kps) {
  __shared__ float4 lds[DotLds<MR>::FLOAT4S];
  skinny_dot_block<MR, NC>(A, B, out, M, N, K, kps, blockIdx.x, blockIdx.y, gridDim.y, lds);
}

template <int KR, bool TA, bool TB>
__global__ void __launch_bounds__(256) k_gemm_outer(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M,
                                                    int N, int K, int rows_per_wave) {
  outer_block<KR, TA, TB>(A, B, C, M, N, K, rows_per_wave, blockIdx.x, blockIdx.y);
}

// One streamed product's share of a grouped launch (k_stream_group): which kernel's block code it
// runs, its arguments (`arg`: K split length of the rows and dot kernels, rows per wave of the
// outer product) and its 2-D grid, gx blocks wide.
// A few outputs with a long K (at most 16384 outputs): one block of W waves per output, its
// threads taking k 64 W apart in increasing order (eight loads of each operand in flight), each
// wave's sum by a fixed butterfly, and the W wave sums added in wave order. Any flags, any
// alignment.
//
// Output e of k_gemm_tiny_out<W>, computed by 64 W / V threads: thread t also runs threads
// t + 64 W / V, t + 128 W / V, ... of the W-wave block (V of them in all), with the same loads,
// sums and order, so that a grouped launch of 256-thread blocks gives the single kernel's bits.
template <int W, int V>
__device__ __forceinline__ void tiny_block(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N,
                                           int K, bool ta, bool tb, uint32_t e, float* wsum) {
  constexpr int NT = 64 * W, RT = NT / V;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int i = e / N, j = e % N;
  float sum[V];
#pragma unroll
  for (int v = 0; v < V; v++) {
    float acc = 0.f;
    int k = threadIdx.x + v * RT;
    for (; k + 7 * NT < K; k += 8 * NT) {
      float a[8], b[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const uint64_t kk = (uint64_t)(k + u * NT);
        a[u] = ta ? A[kk * M + i] : A[(uint64_t)i * K + kk];
        b[u] = tb ? B[(uint64_t)j * K + kk] : B[kk * N + j];
      }
#pragma unroll
      for (int u = 0; u < 8; u++) acc = fmaf(a[u], b[u], acc);
    }
    for (; k < K; k += NT) {
      const float a = ta ? A[(uint64_t)k * M + i] : A[(uint64_t)i * K + k];
      const float b = tb ? B[(uint64_t)j * K + k] : B[(uint64_t)k * N + j];
      acc = fmaf(a, b, acc);
    }
    sum[v] = rg_wave_sum(acc);
  }
  if (W == 1) {
    if (lane == 0) C[e] = sum[0];
    return;
  }
  if (lane == 0)
#pragma unroll
    for (int v = 0; v < V; v++) wsum[w + v * (W / V)] = sum[v];
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = wsum[0];
#pragma unroll
    for (int q = 1; q < W; q++) t += wsum[q];
    C[e] = t;
  }
}

template <int W>
__global__ void __launch_bounds__(64 * W) k_gemm_tiny_out(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M,
                                                          int N, int K, bool ta, bool tb) {
  __shared__ float wsum[W];
  tiny_block<W, 1>(A, B, C, M, N, K, ta, tb, blockIdx.x, wsum);
}

enum StreamKind { STREAM_ROWS8 = 0, STREAM_DOT8, STREAM_OUTER8_TN, STREAM_OUTER8_NT, STREAM_OUTER8_NN, STREAM_TINY4, STREAM_TINY8, STREAM_TINY16 };
struct StreamPart {
  const float *a, *b;
  float* out;
  int m, n, k, arg, kind;
  bool ta, tb;
  uint32_t gx, gy, blocks;
};
struct StreamParts {
  StreamPart p[3];
};

__device__ __forceinline__ void stream_part(const StreamPart& p, uint32_t bid, float4* lds) {
  const uint32_t bx = bid % p.gx, by = bid / p.gx;
  switch (p.kind) {
    case STREAM_ROWS8: skinny_rows_block<8>(p.a, p.b, p.out, p.m, p.n, p.k, p.ta, p.arg, bx, by, lds); break;
    case STREAM_DOT8: skinny_dot_block<8, 4>(p.a, p.b, p.out, p.m, p.n, p.k, p.arg, bx, by, p.gy, lds); break;
    case STREAM_OUTER8_TN: outer_block<8, true, false>(p.a, p.b, p.out, p.m, p.n, p.k, p.arg, bx, by); break;
    case STREAM_OUTER8_NT: outer_block<8, false, true>(p.a, p.b, p.out, p.m, p.n, p.k, p.arg, bx, by); break;
    case STREAM_TINY4: tiny_block<4, 1>(p.a, p.b, p.out, p.m, p.n, p.k, p.ta, p.tb, bid, (float*)lds); break;
    case STREAM_TINY8: tiny_block<8, 2>(p.a, p.b, p.out, p.m, p.n, p.k, p.ta, p.tb, bid, (float*)lds); break;
    case STREAM_TINY16: tiny_block<16, 4>(p.a, p.b, p.out, p.m, p.n, p.k, p.ta, p.tb, bid, (float*)lds); break;
    default: outer_block<8, false, false>(p.a, p.b, p.out, p.m, p.n, p.k, p.arg, bx, by); break;
  }
}

// Up to three independent streamed products of at most 8 rows (or K at most 8), or of a few
// outputs with a long K, in one launch: part i takes the next p[i].blocks blocks and runs its own
// kernel's block code, with one LDS buffer. The reads of one product and the writes of another share HBM in the same launch, and
// the launch's fixed cost is paid once.
__global__ void __launch_bounds__(256) k_stream_group(StreamParts g) {
  constexpr int F = RowsLds<8>::FLOAT4S > DotLds<8>::FLOAT4S ? RowsLds<8>::FLOAT4S : DotLds<8>::FLOAT4S;
  __shared__ float4 lds[F];
  uint32_t bid = blockIdx.x;
  if (bid < g.p[0].blocks) return stream_part(g.p[0], bid, lds);
  bid -= g.p[0].blocks;
  if (bid < g.p[1].blocks) return stream_part(g.p[1], bid, lds);
  stream_part(g.p[2], bid - g.p[1].blocks, lds);
}

enum SkinnyKind { SKINNY_NONE = 0, SKINNY_ROWS, SKINNY_DOT, SKINNY_OUTER, SKINNY_TINY };

// A skinny product as one of the kernels sees it. A matrix-vector product (n == 1) is run as its
// transpose, C^T = op(B)^T op(A)^T: with one column, C and C^T are the same memory, and the
// streamed matrix becomes the kernels' right operand.
struct Skinny {
  SkinnyKind kind = SKINNY_NONE;
  bool swapped = false;  // roles of A and B exchanged (n == 1)
  uint64_t m = 0, n = 0, k = 0;
  bool ta = false;
};

bool use_mfma(int dtype, uint64_t m, uint64_t n, uint64_t k) {
  return dtype == RG_F32 && m >= 32 && n >= 32 && k >= 8 && m * n * k >= (1u << 18);
}

// Which skinny kernel a product takes, from shapes and flags alone (alignment is checked at
// launch; an unaligned operand falls back to the general kernels).
Skinny skinny_plan(int dtype, uint64_t m, uint64_t n, uint64_t k, uint64_t batch, bool ta, bool tb) {
  Skinny sk;
  if (dtype != RG_F32 || batch != 1 || m == 0 || n == 0 || k == 0) return sk;
  sk.m = m;
  sk.n = n;
  sk.k = k;
  sk.ta = ta;
  if (k <= 16 && n % 4 == 0 && m * n >= (1ull << 14)) {
    sk.kind = SKINNY_OUTER;
    return sk;
  }
  if (m <= 16 && k >= 512 && n >= 64) {
    if (!tb && n % 4 == 0) sk.kind = SKINNY_ROWS;
    else if (tb && !ta && k % 256 == 0 && n % 4 == 0) sk.kind = SKINNY_DOT;
    if (sk.kind != SKINNY_NONE) return sk;
  }
  if (n == 1 && k >= 512 && m >= 64) {
    // op(A) x with A stored K x M (ta): rows kernel over A; stored M x K: dot kernel over A's rows.
    sk.swapped = true;
    sk.m = 1;
    sk.n = m;
    sk.ta = false;
    if (ta && m % 4 == 0) sk.kind = SKINNY_ROWS;
    else if (!ta && k % 256 == 0 && m % 4 == 0) sk.kind = SKINNY_DOT;
    if (sk.kind != SKINNY_NONE) return sk;
    sk = Skinny{};
  }
  // Outputs with both sides at least 32 (a tied embedding's gradient, 96 x 128 over 4096 rows)
  // go to the MFMA tiles, which read both operands in coalesced tiles.
  if (m * n <= 16384 && k >= 512 && !use_mfma(dtype, m, n, k)) {
    sk = Skinny{};
    sk.kind = SKINNY_TINY;
    sk.m = m;
    sk.n = n;
    sk.k = k;
    sk.ta = ta;
  }
  return sk;
}

// K split length of SKINNY_DOT: the whole K in chunks of at most DOT_KPS (1024, or 512 for 16
// rows, whose panel would not fit), each a multiple of 256.
int skinny_dot_kps(uint64_t m, uint64_t k) {
  const uint64_t cap = m <= 8 ? DOT_KPS : DOT_KPS / 2;
  const uint64_t splits = (k + cap - 1) / cap;
  return (int)(((k + splits - 1) / splits + 255) / 256 * 256);
}

// K splits of SKINNY_ROWS: about 1024 waves, each at least 64 rows of K deep, at most 16.
int skinny_rows_splits(uint64_t n, uint64_t k) {
  const uint64_t blocks = (n + 255) / 256;
  uint64_t want = (256 + blocks - 1) / blocks;
  const uint64_t most = std::max<uint64_t>(1, k / 256);
  return (int)std::max<uint64_t>(1, std::min<uint64_t>(std::min(want, most), 16));
}

struct TileCfg {
  int bm, bn, bk, wm, wn, ms = 16;
};

int split_count(const TileCfg& t, uint64_t m, uint64_t n, uint64_t k, uint64_t batch);

// Block tile, from measurements of C4's products on MI355X: 32-wide tiles for outputs 32..96 wide
// or 32 tall (attention heads, the vocabulary); 128x128 when that still yields two blocks per CU
// (512), then 128x64 at two blocks per CU; 128x64 with eight waves (two per SIMD) at one block per
// CU, and for long-K products with at least 32 such tiles (split over K to 256 blocks); 64x128 at
// one block per CU; 64x64 (split over K when that leaves the CUs idle); 32x32 when even split
// 64x64 tiles come to fewer than 256 blocks (C3's products). The same shapes whichever operand is
// K-contiguous: with the non-temporal output stores, 64x64 tiles of 32x32 MFMAs, once faster for a
// K-contiguous B, are 1-9 % slower than 128x64 ones on C4's input-gradient products.
TileCfg pick_tile(uint64_t m, uint64_t n, uint64_t k, uint64_t batch) {
  auto blocks = [&](int bm, int bn) { return ((m + bm - 1) / bm) * ((n + bn - 1) / bn) * batch; };
  if (n <= 96 && n % 32 == 0) return {128, 32, 32, 4, 1};
  if (m <= 32) return {32, 128, 32, 1, 4};
  if (blocks(128, 128) >= 512) return {128, 128, 16, 2, 2};
  if (blocks(128, 64) >= 512) return {128, 64, 16, 2, 2};
  if (blocks(128, 64) >= 256 || (blocks(128, 64) >= 32 && k >= 4096)) return {128, 64, 32, 2, 4};
  if (blocks(64, 128) >= 256) return {64, 128, 32, 2, 2};
  // Small outputs: 32x32 tiles when 64x64 ones, split over K where K allows, would leave most
  // CUs idle (C3's products: 4096 x 128 over K <= 512, 128 x 128 weight gradients).
  const TileCfg t64 = {64, 64, 32, 2, 2};
  if (blocks(64, 64) * (uint64_t)split_count(t64, m, n, k, batch) < 256) return {32, 32, 32, 2, 2};
  return t64;
}

// K splits for products with too few tiles: about 256 blocks of eight waves or 768 of four, each
// split at least 512 deep, at most 16.
int split_count(const TileCfg& t, uint64_t m, uint64_t n, uint64_t k, uint64_t batch) {
  uint64_t tiles = ((m + t.bm - 1) / t.bm) * ((n + t.bn - 1) / t.bn) * batch;
  if (tiles >= 256 || k < 1024) return 1;
  uint64_t target = t.wm * t.wn == 8 ? 256 : 768;
  uint64_t want = (target + tiles - 1) / tiles;
  uint64_t most = k / 512;
  return (int)std::max<uint64_t>(1, std::min<uint64_t>(std::min(want, most), 16));
}

struct Launch {
  dim3 grid;
  const float *a, *b;
  float* c;
  int m, n, k;
  const int64_t *a_off, *b_off;
  uint64_t as, bs;
  int splits, kps;
  float* part;
  const float* bias;
  uint32_t tm, tn;
};

template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, int MS>
void launch_mode(hipStream_t s, int mode, const Launch& l) {
#define RG_GEMM(MODE_)                                                                                                       \
  hipLaunchKernelGGL((k_gemm_mfma<BM, BN, BK, WM, WN, TA, TB, MODE_, MS>), l.grid, dim3(64 * WM * WN), 0, s, l.a, l.b, l.c, l.m, l.n, \
                     l.k, l.a_off, l.b_off, l.as, l.bs, l.splits, l.kps, l.part, l.bias, l.tm, \
                     l.tn, 1)
  if (mode == LOAD_EVEN) RG_GEMM(LOAD_EVEN);
  else if (mode == LOAD_VEC) RG_GEMM(LOAD_VEC);
  else RG_GEMM(LOAD_SCALAR);
#undef RG_GEMM
}

template <int BM, int BN, int BK, int WM, int WN, int MS = 16>
void launch_flags(hipStream_t s, bool ta, bool tb, int mode, const Launch& l) {
  if (!ta && !tb) launch_mode<BM, BN, BK, WM, WN, false, false, MS>(s, mode, l);
  else if (ta && !tb) launch_mode<BM, BN, BK, WM, WN, true, false, MS>(s, mode, l);
  else if (!ta && tb) launch_mode<BM, BN, BK, WM, WN, false, true, MS>(s, mode, l);
  else launch_mode<BM, BN, BK, WM, WN, true, true, MS>(s, mode, l);
}

// Instantiates the tile shapes pick_tile can return.
void launch_mfma(hipStream_t s, const TileCfg& t, bool ta, bool tb, int mode, const Launch& l) {
#define RG_TILE(BM_, BN_, BK_, WM_, WN_) \
  if (t.bm == BM_ && t.bn == BN_ && t.bk == BK_ && t.wm == WM_ && t.wn == WN_ && t.ms == 16) return launch_flags<BM_, BN_, BK_, WM_, WN_>(s, ta, tb, mode, l)
  RG_TILE(128, 128, 16, 2, 2);
  RG_TILE(128, 64, 16, 2, 2);
  RG_TILE(128, 64, 32, 2, 4);
  RG_TILE(64, 128, 32, 2, 2);
  RG_TILE(64, 64, 32, 2, 2);
  RG_TILE(128, 32, 32, 4, 1);
  RG_TILE(32, 128, 32, 1, 4);
  RG_TILE(32, 32, 32, 2, 2);
#undef RG_TILE
}

}  // namespace

bool gemm_streamed(int dtype, uint64_t m, uint64_t n, uint64_t k, uint64_t batch, bool ta, bool tb) {
  return skinny_plan(dtype, m, n, k, batch, ta, tb).kind != SKINNY_NONE;
}

int gemm_splits(int dtype, uint64_t m, uint64_t n, uint64_t k, uint64_t batch, bool ta, bool tb) {
  if (m == 0 || n == 0 || batch == 0) return 1;
  const Skinny sk = skinny_plan(dtype, m, n, k, batch, ta, tb);
  if (sk.kind == SKINNY_ROWS) {
    const int splits = skinny_rows_splits(sk.n, sk.k);
    const uint64_t kps = (sk.k + splits - 1) / splits;
    return (int)((sk.k + kps - 1) / kps);
  }
  if (sk.kind == SKINNY_DOT) {
    const uint64_t kps = (uint64_t)skinny_dot_kps(sk.m, sk.k);
    return (int)((sk.k + kps - 1) / kps);
  }
  if (sk.kind != SKINNY_NONE || !use_mfma(dtype, m, n, k)) return 1;
  TileCfg t = pick_tile(m, n, k, batch);
  int splits = split_count(t, m, n, k, batch);
  uint64_t kps = ((k + splits - 1) / splits + t.bk - 1) / t.bk * t.bk;
  return (int)((k + kps - 1) / kps);
}

bool gemm_epilogue_tile(int dtype, uint64_t m, uint64_t n, uint64_t k, bool ta, bool tb, GemmTile* out) {
  if (m == 0 || n == 0 || m >= (1ull << 31) || n >= (1ull << 31) || k >= (1ull << 31)) return false;
  if (skinny_plan(dtype, m, n, k, 1, ta, tb).kind != SKINNY_NONE || !use_mfma(dtype, m, n, k)) return false;
  TileCfg t = pick_tile(m, n, k, 1);
  // Short K: 128x64 tiles rather than 128x128, twice the blocks, so that the second round's
  // products run while the first round's epilogues read and write (C4's GELU backward: 3 % off
  // the combined kernels on MI355X, results unchanged).
  if (t.bm == 128 && t.bn == 128 && k <= 1024) t = TileCfg{128, 64, 16, 2, 2};
  if (split_count(t, m, n, k, 1) != 1) return false;
  // Runs of adjacent output columns per lane: four with a K-contiguous B (the transposed product
  // form); with an N-contiguous B one per tile the wave holds across N, which must be two or four.
  if (!tb && (t.bn / t.wn) / t.ms != 4 && (t.bn / t.wn) / t.ms != 2) return false;
  const bool vec = k % 4 == 0 && (!ta || m % 4 == 0) && (tb || n % 4 == 0) && n % 4 == 0;
  if (!vec) return false;
  const bool even = m % t.bm == 0 && n % t.bn == 0 && k % t.bk == 0;
  *out = GemmTile{t.bm, t.bn, t.bk, t.wm, t.wn, t.ms, even ? LOAD_EVEN : LOAD_VEC, (int)((k + t.bk - 1) / t.bk * t.bk),
                  (uint32_t)((m + t.bm - 1) / t.bm), (uint32_t)((n + t.bn - 1) / t.bn)};
  return true;
}

uint64_t gemm_workspace(int dtype, uint64_t m, uint64_t n, uint64_t k, uint64_t batch, bool ta, bool tb) {
  int s = gemm_splits(dtype, m, n, k, batch, ta, tb);
  return s > 1 ? (uint64_t)s * batch * m * n * sizeof(float) : 0;
}

// Launches the skinny kernel of `sk`; false when an operand is not aligned for it.
bool gemm_skinny(hipStream_t s, const GemmArgs& g, const Skinny& sk) {
  auto aligned = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  if (g.bias || g.a_off || g.b_off || !aligned(g.c)) return false;
  // With the roles exchanged (n == 1) the vector is the left operand of one row.
  const float* A = (const float*)(sk.swapped ? g.b : g.a);
  const float* B = (const float*)(sk.swapped ? g.a : g.b);
  float* C = (float*)g.c;
  const int M = (int)sk.m, N = (int)sk.n, K = (int)sk.k;
  const SkinnyKind kind = sk.kind;
  if (g.defer_split && (kind == SKINNY_TINY || kind == SKINNY_OUTER))
    throw std::runtime_error("deferred K-split product on a kernel that does not split K");
  if (kind == SKINNY_TINY) {
    // Waves per output: enough that each thread's share of K is one batch of eight loads.
    const dim3 grid((uint32_t)(M * N));
    const int w = std::min(16, std::max(1, (K + 511) / 512));
    if (w <= 1) hipLaunchKernelGGL(k_gemm_tiny_out<1>, grid, dim3(64), 0, s, A, B, C, M, N, K, g.ta, g.tb);
    else if (w <= 2) hipLaunchKernelGGL(k_gemm_tiny_out<2>, grid, dim3(128), 0, s, A, B, C, M, N, K, g.ta, g.tb);
    else if (w <= 4) hipLaunchKernelGGL(k_gemm_tiny_out<4>, grid, dim3(256), 0, s, A, B, C, M, N, K, g.ta, g.tb);
    else if (w <= 8) hipLaunchKernelGGL(k_gemm_tiny_out<8>, grid, dim3(512), 0, s, A, B, C, M, N, K, g.ta, g.tb);
    else hipLaunchKernelGGL(k_gemm_tiny_out<16>, grid, dim3(1024), 0, s, A, B, C, M, N, K, g.ta, g.tb);
    return true;
  }
  if (kind == SKINNY_OUTER) {
    // 16 rows per wave for tall outputs; fewer for short ones, so more waves share the work.
    const int rows = std::max(1, std::min(16, M / 256));
    dim3 grid((uint32_t)((N + 255) / 256), (uint32_t)((M + 4 * rows - 1) / (4 * rows)));
    if (!g.tb && !aligned(B)) return false;
#define RG_OUTER_K(KR_, TA_, TB_) hipLaunchKernelGGL((k_gemm_outer<KR_, TA_, TB_>), grid, dim3(256), 0, s, A, B, C, M, N, K, rows)
#define RG_OUTER(TA_, TB_)                   \
  do {                                       \
    if (K <= 1) RG_OUTER_K(1, TA_, TB_);     \
    else if (K <= 4) RG_OUTER_K(4, TA_, TB_); \
    else if (K <= 8) RG_OUTER_K(8, TA_, TB_); \
    else RG_OUTER_K(16, TA_, TB_);           \
  } while (0)
    if (g.ta && g.tb) RG_OUTER(true, true);
    else if (g.ta) RG_OUTER(true, false);
    else if (g.tb) RG_OUTER(false, true);
    else RG_OUTER(false, false);
#undef RG_OUTER
#undef RG_OUTER_K
    return true;
  }
  // Both K-split kernels leave split s's partials at [s][M N] of the workspace; the split sum (or
  // the deferred fold_wide) adds them in split order.
  auto sum_splits = [&](const float* part, int splits) {
    if (g.defer_split && splits != g.planned_splits)
      throw std::runtime_error("deferred K-split product: " + std::to_string(splits) + " streamed partial products, the fold expects " +
                               std::to_string(g.planned_splits));
    if (splits > 1 && !g.defer_split) {
      const uint64_t mn = g.m * g.n;
      hipLaunchKernelGGL(k_split_sum, dim3((uint32_t)((mn + 1023) / 1024), 1), dim3(256), 0, s, part, C, mn, splits, (const float*)nullptr, g.n);
    }
  };
  if (kind == SKINNY_DOT) {
    if (!aligned(A) || !aligned(B)) return false;
    constexpr int NC = 4;
    const int kps = skinny_dot_kps(sk.m, sk.k);
    const int splits = (K + kps - 1) / kps;
    float* out = splits > 1 ? (float*)g.workspace : C;
    dim3 grid((uint32_t)((N + 4 * NC - 1) / (4 * NC)), (uint32_t)splits);
    if (M <= 8) hipLaunchKernelGGL((k_gemm_skinny_dot<8, NC>), grid, dim3(256), 0, s, A, B, out, M, N, K, kps);
    else hipLaunchKernelGGL((k_gemm_skinny_dot<16, NC>), grid, dim3(256), 0, s, A, B, out, M, N, K, kps);
    sum_splits(out, splits);
    return true;
  }
  if (!aligned(B)) return false;
  const int splits0 = skinny_rows_splits(sk.n, sk.k);
  const int kps = (K + splits0 - 1) / splits0;
  const int splits = (K + kps - 1) / kps;
  float* out = splits > 1 ? (float*)g.workspace : C;
  dim3 grid((uint32_t)((N + 255) / 256), (uint32_t)splits);
  if (M <= 8) hipLaunchKernelGGL((k_gemm_skinny_rows<8, 8>), grid, dim3(256), 0, s, A, B, out, M, N, K, sk.ta, kps);
  else hipLaunchKernelGGL((k_gemm_skinny_rows<16, 8>), grid, dim3(256), 0, s, A, B, out, M, N, K, sk.ta, kps);
  sum_splits(out, splits);
  return true;
}

namespace {

// The MFMA tile launch of product `g`: its tile, load mode and launch arguments.
void mfma_launch(const GemmArgs& g, TileCfg* tile, int* load_mode, Launch* launch) {
  TileCfg t = pick_tile(g.m, g.n, g.k, g.batch);
  int splits = split_count(t, g.m, g.n, g.k, g.batch);
  int kps = (int)(((g.k + splits - 1) / splits + t.bk - 1) / t.bk * t.bk);
  splits = (int)((g.k + kps - 1) / kps);
  if (g.defer_split && splits != g.planned_splits)
    throw std::runtime_error("deferred K-split product: " + std::to_string(splits) + " partial products, the fold expects " +
                             std::to_string(g.planned_splits));
  // 16-byte vector loads need 16-byte aligned operand rows: aligned bases, leading dimensions
  // (K, or M / N for the contiguous-column layouts) and batch offsets that are multiples of 4.
  auto aligned = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  bool vec = aligned(g.a) && aligned(g.b) && g.k % 4 == 0 && (!g.ta || g.m % 4 == 0) && (g.tb || g.n % 4 == 0) &&
             (g.a_off ? g.a_off4 : g.a_stride % 4 == 0) && (g.b_off ? g.b_off4 : g.b_stride % 4 == 0);
  bool even = g.m % t.bm == 0 && g.n % t.bn == 0 && g.k % t.bk == 0 && kps % t.bk == 0;
  int mode = !vec ? LOAD_SCALAR : even ? LOAD_EVEN : LOAD_VEC;
  Launch l;
  l.tm = (uint32_t)((g.m + t.bm - 1) / t.bm);
  l.tn = (uint32_t)((g.n + t.bn - 1) / t.bn);
  l.grid = dim3((uint32_t)(l.tm * l.tn * g.batch * splits));
  l.a = (const float*)g.a;
  l.b = (const float*)g.b;
  l.c = (float*)g.c;
  l.m = (int)g.m;
  l.n = (int)g.n;
  l.k = (int)g.k;
  l.a_off = g.a_off;
  l.b_off = g.b_off;
  l.as = g.a_stride;
  l.bs = g.b_stride;
  l.splits = splits;
  l.kps = kps;
  l.part = splits > 1 ? (float*)g.workspace : nullptr;
  l.bias = splits > 1 ? nullptr : (const float*)g.bias;
  *tile = t;
  *load_mode = mode;
  *launch = l;
}

// Whether product `g` goes to the MFMA tiles (not a streaming kernel, not the plain kernel).
bool on_mfma_tiles(const GemmArgs& g) {
  return g.m && g.n && g.batch && skinny_plan(g.dtype, g.m, g.n, g.k, g.batch, g.ta, g.tb).kind == SKINNY_NONE &&
         use_mfma(g.dtype, g.m, g.n, g.k);
}

}  // namespace

// Plan slots start 256-byte aligned, so a lowered product always meets the skinny kernels'
// alignment. A product whose K-split partials are deferred to the fold area must leave exactly
// the planned number of partial products there: a launch that would take another path (the
// streaming kernel refusing its operands, another split count) throws instead, and the error is
// latched like any failed launch, rather than letting the fold overwrite C with stale partials.
void gemm(hipStream_t s, const GemmArgs& g) {
  if (g.m == 0 || g.n == 0 || g.batch == 0) return;
  const Skinny sk = skinny_plan(g.dtype, g.m, g.n, g.k, g.batch, g.ta, g.tb);
  if (sk.kind != SKINNY_NONE) {
    if (gemm_skinny(s, g, sk)) return;
    if (g.defer_split) throw std::runtime_error("deferred K-split product: the streaming kernel refused its operands");
  }
  if (use_mfma(g.dtype, g.m, g.n, g.k)) {
    TileCfg t;
    int mode;
    Launch l;
    mfma_launch(g, &t, &mode, &l);
    const int splits = l.splits;
    launch_mfma(s, t, g.ta, g.tb, mode, l);
    if (splits > 1 && !g.defer_split) {
      uint64_t mn = g.m * g.n;
      hipLaunchKernelGGL(k_split_sum, dim3((uint32_t)((mn + 1023) / 1024), (uint32_t)g.batch), dim3(256), 0, s, (const float*)l.part,
                         (float*)g.c, mn, splits, (const float*)g.bias, g.n);
    }
    return;
  }
  if (g.defer_split) throw std::runtime_error("deferred K-split product on the plain kernel, which does not split K");
  dim3 grid((uint32_t)((g.m * g.n + 255) / 256), (uint32_t)g.batch);
  if (g.dtype == RG_F32)
    hipLaunchKernelGGL(k_gemm_plain<float>, grid, dim3(256), 0, s, (const float*)g.a, (const float*)g.b, (float*)g.c, (uint32_t)g.m,
                       (uint32_t)g.n, (uint32_t)g.k, g.ta, g.tb, g.a_off, g.b_off, g.a_stride, g.b_stride);
  else
    hipLaunchKernelGGL(k_gemm_plain<double>, grid, dim3(256), 0, s, (const double*)g.a, (const double*)g.b, (double*)g.c, (uint32_t)g.m,
                       (uint32_t)g.n, (uint32_t)g.k, g.ta, g.tb, g.a_off, g.b_off, g.a_stride, g.b_stride);
  if (g.bias && g.dtype == RG_F32) {
    const uint64_t total = g.m * g.n * g.batch;
    hipLaunchKernelGGL(k_add_bias, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, s, (float*)g.c, (const float*)g.bias, total, g.n);
  }
}

namespace {

// Product `g` as a part of a grouped streaming launch: the kernel gemm_skinny would launch for
// it, when that is the row, dot or outer-product kernel for at most 8 rows (or K), or the
// tiny-output kernel of 4, 8 or 16 waves, its operands aligned for it, and its K splits, if any,
// deferred to the fold area.
bool stream_part_of(const GemmArgs& g, StreamPart* p) {
  if (g.m == 0 || g.n == 0 || g.batch != 1 || g.bias || g.a_off || g.b_off) return false;
  auto aligned = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  const Skinny sk = skinny_plan(g.dtype, g.m, g.n, g.k, g.batch, g.ta, g.tb);
  if (!aligned(g.c)) return false;
  const float* A = (const float*)(sk.swapped ? g.b : g.a);
  const float* B = (const float*)(sk.swapped ? g.a : g.b);
  const int M = (int)sk.m, N = (int)sk.n, K = (int)sk.k;
  auto split_ok = [&](int splits) {
    if (splits > 1 && !g.defer_split) return false;
    return !g.defer_split || splits == g.planned_splits;
  };
  StreamPart q{A, B, (float*)g.c, M, N, K, 0, 0, sk.ta, g.tb, 0, 0, 0};
  if (sk.kind == SKINNY_TINY) {
    // k_gemm_tiny_out of 4, 8 or 16 waves (fewer do not fill a 256-thread block).
    const int w = std::min(16, std::max(1, (K + 511) / 512));
    if (w < 3 || g.defer_split) return false;
    q.kind = w <= 4 ? STREAM_TINY4 : w <= 8 ? STREAM_TINY8 : STREAM_TINY16;
    q.ta = g.ta;
    q.gx = (uint32_t)(M * N);
    q.gy = 1;
  } else if (sk.kind == SKINNY_OUTER) {
    if (K > 8 || (!g.tb && !aligned(B)) || (g.ta && g.tb) || g.defer_split) return false;
    q.kind = g.ta ? STREAM_OUTER8_TN : g.tb ? STREAM_OUTER8_NT : STREAM_OUTER8_NN;
    // Half the single kernel's rows per wave, so twice its blocks: 8 rows for C5's 4096-row
    // outputs measured 3 us (4 %) faster per pass on MI355X than 16, and 6 alike, 4 or 32 slower.
    // Each output is one sum either way, so the results do not change.
    q.arg = std::max(1, std::min(8, M / 512));
    q.gx = (uint32_t)((N + 255) / 256);
    q.gy = (uint32_t)((M + 4 * q.arg - 1) / (4 * q.arg));
  } else if (sk.kind == SKINNY_DOT) {
    if (M > 8 || !aligned(A) || !aligned(B)) return false;
    const int kps = skinny_dot_kps(sk.m, sk.k), splits = (K + kps - 1) / kps;
    if (!split_ok(splits)) return false;
    q.kind = STREAM_DOT8;
    q.arg = kps;
    q.out = splits > 1 ? (float*)g.workspace : (float*)g.c;
    q.gx = (uint32_t)((N + 15) / 16);
    q.gy = (uint32_t)splits;
  } else if (sk.kind == SKINNY_ROWS) {
    if (M > 8 || !aligned(B)) return false;
    const int splits0 = skinny_rows_splits(sk.n, sk.k);
    const int kps = (K + splits0 - 1) / splits0, splits = (K + kps - 1) / kps;
    if (!split_ok(splits)) return false;
    q.kind = STREAM_ROWS8;
    q.arg = kps;
    q.out = splits > 1 ? (float*)g.workspace : (float*)g.c;
    q.gx = (uint32_t)((N + 255) / 256);
    q.gy = (uint32_t)splits;
  } else {
    return false;
  }
  q.blocks = q.gx * q.gy;
  *p = q;
  return true;
}

}  // namespace

bool gemm_group(hipStream_t s, const GemmArgs* g, int count, bool launch) {
  if (count < 2 || count > GROUP_MAX) return false;
  {
    // Streamed products (C5's chain): any mix of the row, dot, outer-product and tiny-output kernels.
    StreamParts parts{};
    uint32_t blocks = 0;
    bool all = true;
    for (int i = 0; i < count && all; i++) {
      all = stream_part_of(g[i], &parts.p[i]);
      blocks += all ? parts.p[i].blocks : 0;
    }
    if (all) {
      if (launch) hipLaunchKernelGGL(k_stream_group, dim3(blocks), dim3(256), 0, s, parts);
      return true;
    }
  }
  TileCfg t[GROUP_MAX];
  int mode[GROUP_MAX];
  Launch l[GROUP_MAX];
  int flags = 0;
  for (int i = 0; i < count; i++) {
    if (!on_mfma_tiles(g[i]) || g[i].batch != 1) return false;
    mfma_launch(g[i], &t[i], &mode[i], &l[i]);
    // K-split partials, if any, must be the deferred kind: a split sum after the grouped launch
    // would be a second launch anyway.
    if (l[i].splits > 1 && !g[i].defer_split) return false;
    if (mode[i] != LOAD_EVEN || t[i].bm != t[0].bm || t[i].bn != t[0].bn || t[i].bk != t[0].bk || t[i].wm != t[0].wm ||
        t[i].wn != t[0].wn || t[i].ms != 16 || (i + 1 < count && l[i].grid.x % 8 != 0))
      return false;
    flags |= ((g[i].ta ? 2 : 0) | (g[i].tb ? 1 : 0)) << (2 * i);
  }
  // The shapes and flag sequences instantiated, from C4's backward pass: on 128x64 tiles of
  // eight waves, fc1's input and weight gradients as a pair, with fc2's weight gradient ahead of
  // them as a triple; on 64x64 tiles of four waves, the attention projection's weight gradient
  // with the q, k, v projection's.
  constexpr int T = 2, N = 1;  // (ta, tb) = (true, false) and (false, true)
  const bool wide = t[0].bm == 128 && t[0].bn == 64 && t[0].bk == 32 && t[0].wm == 2 && t[0].wn == 4;
  const bool small = t[0].bm == 64 && t[0].bn == 64 && t[0].bk == 32 && t[0].wm == 2 && t[0].wn == 2;
  const bool known = (wide && ((count == 2 && (flags == (N | T << 2) || flags == (T | N << 2))) ||
                               (count == 3 && flags == (T | N << 2 | T << 4)))) ||
                     (small && count == 2 && flags == (T | T << 2));
  if (!launch || !known) return known;
  GroupParts parts{};
  uint32_t blocks = 0;
  for (int i = 0; i < count; i++) {
    parts.p[i] = GroupPart{l[i].a, l[i].b, l[i].c, l[i].part, l[i].bias, l[i].m, l[i].n, l[i].k, l[i].splits, l[i].kps, l[i].tm, l[i].tn,
                           l[i].grid.x};
    blocks += l[i].grid.x;
  }
  const dim3 grid(blocks);
  if (small)
    hipLaunchKernelGGL((k_gemm_mfma_group<64, 64, 32, 2, 2, 2, T | T << 2>), grid, dim3(256), 0, s, parts);
  else if (count == 2 && flags == (N | T << 2))
    hipLaunchKernelGGL((k_gemm_mfma_group<128, 64, 32, 2, 4, 2, N | T << 2>), grid, dim3(512), 0, s, parts);
  else if (count == 2)
    hipLaunchKernelGGL((k_gemm_mfma_group<128, 64, 32, 2, 4, 2, T | N << 2>), grid, dim3(512), 0, s, parts);
  else
    hipLaunchKernelGGL((k_gemm_mfma_group<128, 64, 32, 2, 4, 3, T | N << 2 | T << 4>), grid, dim3(512), 0, s, parts);
  return true;
}

}  // namespace rgk
