// The fp32 MFMA product tile (`gemm_mfma_block`) and what it is built from, shared by the
// precompiled product kernels (gemm.hip, where every tile shape and the plain epilogue are
// instantiated) and by the JIT-compiled products whose epilogue applies the elementwise group
// that reads the product (jit.cpp: the same tile, the group's operations applied to each finished
// output before it is stored). Self-contained device code: no includes, so that hiprtc can
// compile it from its text (rg_gemm_mfma_source).
#pragma once

namespace rgg {

#if defined(__HIPCC_RTC__)
// hiprtc declares the fixed-width integer types in its own namespace.
typedef __hip_internal::int64_t int64_t;
typedef __hip_internal::uint64_t uint64_t;
typedef __hip_internal::uint32_t uint32_t;
#endif

template <int V>
struct IC {
  static constexpr int value = V;
};

typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int64_t batch_offset(const int64_t* offs, uint64_t stride, uint32_t b) {
  return offs ? offs[b] : (int64_t)(stride * b);
}

// Which output tile a block computes. The dispatcher deals consecutive blocks round-robin over
// the 8 XCDs, each with its own L2; with `swizzle`, XCD x instead receives the contiguous run
// x*nb/8 ... (x+1)*nb/8 - 1 of tiles, and within a batch the tiles run in groups of 8 M-panels
// per N sweep, so blocks resident on one XCD share their A and B panels in its L2.
struct TileIndex {
  uint32_t tm, tn, z;
};

// Block `bid` of a product launched as `nb` blocks (its share of the grid).
__device__ __forceinline__ TileIndex tile_of(uint32_t bid, uint32_t nb, uint32_t tiles_m, uint32_t tiles_n, int swizzle) {
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

typedef float floatx16 __attribute__((ext_vector_type(16)));

// One MFMA step of shape MS x MS (16x16x4 or 32x32x2 f32): lane l supplies row (A) / column (B)
// l % MS at k = l / MS, and register r of its accumulator holds row 8 (r / 4) + 4 (l / MS) + r % 4,
// column l % MS.
template <int MS>
struct Mfma;
template <>
struct Mfma<16> {
  typedef floatx4 acc_t;
  static constexpr int REGS = 4;
  static __device__ __forceinline__ acc_t step(float a, float b, acc_t c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }
};
template <>
struct Mfma<32> {
  typedef floatx16 acc_t;
  static constexpr int REGS = 16;
  static __device__ __forceinline__ acc_t step(float a, float b, acc_t c) { return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0); }
};

// Load modes: every vector inside the operand (no checks), checked 16-byte vectors, or checked
// scalar loads (operands whose rows are not 16-byte aligned).
enum LoadMode { LOAD_EVEN = 0, LOAD_VEC = 1, LOAD_SCALAR = 2 };

// Stages an R x W tile (W contiguous floats per row, W % 4 == 0) of a row-major operand with
// leading dimension `ld`, rows r0.. (valid below `rows`) and columns c0.. (valid below `cols`),
// through registers: NT threads, one 4-float vector per thread and pass.
template <int R, int W, int NT, int MODE>
struct Stager {
  static constexpr int NVEC = R * W / 4;
  static constexpr int PER = (NVEC + NT - 1) / NT;
  float4 v[PER];
  __device__ __forceinline__ void load(const float* base, int64_t ld, int r0, int c0, int rows, int cols, int tid) {
#pragma unroll
    for (int q = 0; q < PER; q++) {
      const int idx = q * NT + tid;
      const int r = idx / (W / 4), c = (idx % (W / 4)) * 4;
      const bool live = NVEC % NT == 0 || idx < NVEC;
      const int gr = r0 + r, gc = c0 + c;
      if constexpr (MODE == LOAD_SCALAR) {
        const float* p = base + (int64_t)gr * ld + gc;
        float t[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          bool ok = live && gr < rows && gc + e < cols;
          t[e] = ok ? p[e] : 0.0f;
        }
        v[q] = make_float4(t[0], t[1], t[2], t[3]);
      } else {
        const bool ok = live && (MODE == LOAD_EVEN || (gr < rows && gc < cols));
        const float4 x = *(const float4*)(ok ? base + (int64_t)gr * ld + gc : base);
        v[q] = ok ? x : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  }
  __device__ __forceinline__ void store(float* lds, int ldl, int tid) const {
#pragma unroll
    for (int q = 0; q < PER; q++) {
      const int idx = q * NT + tid;
      if (NVEC % NT == 0 || idx < NVEC) *(float4*)(lds + (idx / (W / 4)) * ldl + (idx % (W / 4)) * 4) = v[q];
    }
  }
};

template <int T>
__device__ __forceinline__ void lds_read(const float* p, float* v) {
  if constexpr (T == 1) {
    v[0] = *p;
  } else if constexpr (T == 2) {
    float2 x = *(const float2*)p;
    v[0] = x.x; v[1] = x.y;
  } else {
    float4 x = *(const float4*)p;
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
  }
}

// C = op(A) op(B) for one BM x BN block tile; WM x WN wave64s, each owning (BM/WM) x (BN/WN) as
// TM x TN MFMA tiles of 16x16. The grid is one-dimensional: tiles_m * tiles_n * batch * splits
// blocks (tile_of); split `sp` covers K range [sp * k_per_split, (sp + 1) * k_per_split).

// The plain epilogue: each finished output (flat index `e` within the block's output matrix) is
// stored into C, or into the block's split of the K-split partials. Non-temporal stores: every
// block writes its whole tile at the end, all at once; written past the L2 they leave less for the
// end of the kernel to write back (4-10 % off C4's products with 1024- and 768-wide outputs on
// MI355X, results unchanged).
struct StoreC {
  float* C;
  float* partial;
  int splits;
  uint64_t mn;
  float* out = nullptr;
  __device__ __forceinline__ void begin(uint32_t b, uint32_t sp) {
    out = splits > 1 ? partial + ((uint64_t)b * splits + sp) * mn : C + (uint64_t)b * mn;
  }
  __device__ __forceinline__ void put4(uint64_t e, float4 v, int) { __builtin_nontemporal_store(floatx4{v.x, v.y, v.z, v.w}, (floatx4*)(out + e)); }
  __device__ __forceinline__ void put2(uint64_t e, float2 v) { __builtin_nontemporal_store(floatx2{v.x, v.y}, (floatx2*)(out + e)); }
  __device__ __forceinline__ void put1(uint64_t e, float v) { __builtin_nontemporal_store(v, out + e); }
};

// LDS of one tile: two buffers of each operand's K step, in the operand's own layout (rows padded
// by 4 floats where K is contiguous).
template <int BM, int BN, int BK, bool TA, bool TB>
struct TileLds {
  static constexpr int LDA = !TA ? BK + 4 : BM, LDB = TB ? BK + 4 : BN;
  static constexpr int SA = !TA ? BM * LDA : BK * LDA, SB = TB ? BN * LDB : BK * LDB;
  static constexpr int FLOATS = 2 * (SA + SB);
};

// The tile of block `bid` of a product launched as `nb` blocks, staging through `smem` (at least
// TileLds<...>::FLOATS floats of LDS): a kernel that runs two products side by side gives each
// its share of the grid and the same LDS.
template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, int MODE, int MS, class Epi>
__device__ __forceinline__ void gemm_mfma_tile(const float* __restrict__ A, const float* __restrict__ B, int M, int N, int K,
                                               const int64_t* a_off, const int64_t* b_off, uint64_t a_stride, uint64_t b_stride, int splits,
                                               int k_per_split, const float* __restrict__ bias, uint32_t tiles_m, uint32_t tiles_n,
                                               int swizzle, Epi& epi, uint32_t bid, uint32_t nb, float* smem) {
  constexpr int NT = 64 * WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / MS, TN = WTN / MS;
  static_assert(TM >= 1 && TN >= 1 && TM <= 4 && TN <= 4 && (TM & (TM - 1)) == 0 && (TN & (TN - 1)) == 0, "wave tiles");
  // A group of KG k: four MFMA steps, lane l taking k = 4 (l / MS) + j at step j in both operands.
  constexpr int KG = 4 * (64 / MS);
  static_assert(BK % KG == 0, "K step");
  typedef Mfma<MS> MF;
  constexpr bool AK = !TA, BKC = TB;  // K-contiguous operands
  typedef TileLds<BM, BN, BK, TA, TB> L;
  constexpr int LDA = L::LDA, LDB = L::LDB, SA = L::SA, SB = L::SB;
  float(*As)[SA] = (float(*)[SA])smem;
  float(*Bs)[SB] = (float(*)[SB])(smem + 2 * SA);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const TileIndex ti = tile_of(bid, nb, tiles_m, tiles_n, swizzle);
  const uint32_t b = ti.z / splits, sp = ti.z % splits;
  const int m0 = ti.tm * BM, n0 = ti.tn * BN;
  const float* Ab = A + batch_offset(a_off, a_stride, b);
  const float* Bb = B + batch_offset(b_off, b_stride, b);
  const int kbeg = sp * k_per_split, kend = min(K, kbeg + k_per_split);
  const int nk = (kend - kbeg + BK - 1) / BK;

  // Two register stages: the global loads of tile t + 2 are issued while tile t is multiplied
  // out of LDS and tile t + 1 waits in registers, so each load has two iterations to arrive.
  Stager<AK ? BM : BK, AK ? BK : BM, NT, MODE> sa0, sa1;
  Stager<BKC ? BN : BK, BKC ? BK : BN, NT, MODE> sb0, sb1;
  // The register stage SET (a constant): two variables rather than an array, so that no stage is
  // ever indexed and both stay in registers.
  auto stage_a = [&](auto set) -> auto& {
    if constexpr (decltype(set)::value == 0) return sa0;
    else return sa1;
  };
  auto stage_b = [&](auto set) -> auto& {
    if constexpr (decltype(set)::value == 0) return sb0;
    else return sb1;
  };
  // Tile t of this block's K range into register stage `stage`.
  auto load_tiles = [&](int t, auto stage) __attribute__((always_inline)) {
    auto& xa = stage_a(stage);
    auto& xb = stage_b(stage);
    const int k0 = kbeg + t * BK;
    if (AK) xa.load(Ab, K, m0, k0, M, kend, tid);
    else xa.load(Ab, M, k0, m0, kend, M, tid);
    if (BKC) xb.load(Bb, K, n0, k0, N, kend, tid);
    else xb.load(Bb, N, k0, n0, kend, N, tid);
  };

  typename MF::acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < MF::REGS; r++) acc[i][j][r] = 0.0f;

  if (nk > 0) {
    load_tiles(0, IC<0>());
    load_tiles(min(1, nk - 1), IC<1>());
    sa0.store(As[0], LDA, tid);
    sb0.store(Bs[0], LDB, tid);
  }
  __syncthreads();
  const int li = lane % MS, q4 = (lane / MS) * 4;
  auto multiply = [&](const float* as, const float* bs) __attribute__((always_inline)) {
#pragma unroll
    for (int kg = 0; kg < BK; kg += KG) {
      float a[4][TM], bv[4][TN];  // [k-step][tile]
      if (AK) {
#pragma unroll
        for (int i = 0; i < TM; i++) {
          float v[4];
          lds_read<4>(as + (wm * WTM + i * MS + li) * LDA + kg + q4, v);
#pragma unroll
          for (int j = 0; j < 4; j++) a[j][i] = v[j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; j++) lds_read<TM>(as + (kg + q4 + j) * LDA + wm * WTM + TM * li, a[j]);
      }
      if (BKC) {
#pragma unroll
        for (int i = 0; i < TN; i++) {
          float v[4];
          lds_read<4>(bs + (wn * WTN + i * MS + li) * LDB + kg + q4, v);
#pragma unroll
          for (int j = 0; j < 4; j++) bv[j][i] = v[j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; j++) lds_read<TN>(bs + (kg + q4 + j) * LDB + wn * WTN + TN * li, bv[j]);
      }
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
          for (int n = 0; n < TN; n++) {
            // With a K-contiguous B the product is formed transposed (B supplies the MFMA rows), so
            // that each lane ends up with four adjacent output columns.
            if constexpr (BKC) acc[i][n] = MF::step(bv[j][n], a[j][i], acc[i][n]);
            else acc[i][n] = MF::step(a[j][i], bv[j][n], acc[i][n]);
          }
    }
  };
  // Iteration t multiplies LDS buffer t % 2, whose register stage t % 2 is then free for tile
  // t + 2; tile t + 1 goes from register stage (t + 1) % 2 into the other LDS buffer, which every
  // wave finished reading before the previous barrier. The body has no branches, so the compiler
  // can interleave the loads and address arithmetic with the MFMAs: past the end of the range the
  // last tile is loaded again and stored into the idle buffer, and never read.
  auto iteration = [&](int t, auto parity) __attribute__((always_inline)) {
    constexpr int P = decltype(parity)::value;
    load_tiles(min(t + 2, nk - 1), parity);
    multiply(As[P], Bs[P]);
    stage_a(IC<P ^ 1>()).store(As[P ^ 1], LDA, tid);
    stage_b(IC<P ^ 1>()).store(Bs[P ^ 1], LDB, tid);
    __syncthreads();
  };
  int t = 0;
  for (; t + 1 < nk; t += 2) {
    iteration(t, IC<0>());
    iteration(t + 1, IC<1>());
  }
  if (t < nk) iteration(t, IC<0>());
  // Accumulator register r of lane l holds MFMA row rho(r) = 8 (r / 4) + 4 (l / MS) + r % 4, column
  // l % MS (for the transposed form: output row l % MS, column rho(r)). MFMA tile i row rho is
  // block row MS i + rho (K-contiguous A) or TM rho + i (M-contiguous A); tile n column gamma is
  // block column MS n + gamma (K-contiguous B) or TN gamma + n (N-contiguous B). Either way a lane
  // holds adjacent output columns: four per group of four registers in one tile (K-contiguous B)
  // or one in each of its TN tiles.
  // put4's third argument names which of the lane's runs of four columns it stores (with a
  // K-contiguous B: tile n, register group g; the same for every row the lane stores), so that an
  // epilogue can keep per-column sums in registers.
  epi.begin(b, sp);
  const bool vec_out = MODE != LOAD_SCALAR && N % 4 == 0;
  // A per-column bias (unsplit products only) added to the finished sums, as one fp32 addition.
  if (bias) {
    if constexpr (BKC) {
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int n = 0; n < TN; n++)
#pragma unroll
          for (int g = 0; g < MF::REGS / 4; g++) {
            const int col = n0 + wn * WTN + n * MS + 8 * g + q4;
#pragma unroll
            for (int r = 0; r < 4; r++)
              if (col + r < N) acc[i][n][4 * g + r] += bias[col + r];
          }
    } else {
      const int col = n0 + wn * WTN + TN * li;
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < MF::REGS; r++)
#pragma unroll
          for (int n = 0; n < TN; n++)
            if (col + n < N) acc[i][n][r] += bias[col + n];
    }
  }
  if constexpr (BKC) {
#pragma unroll
    for (int i = 0; i < TM; i++) {
      const int row = m0 + wm * WTM + (AK ? i * MS + li : TM * li + i);
      if (row >= M) continue;
      const uint64_t erow = (uint64_t)row * N;
#pragma unroll
      for (int n = 0; n < TN; n++)
#pragma unroll
        for (int g = 0; g < MF::REGS / 4; g++) {
          const int col = n0 + wn * WTN + n * MS + 8 * g + q4;
          const auto& c = acc[i][n];
          if (vec_out && col + 4 <= N) {
            epi.put4(erow + col, make_float4(c[4 * g], c[4 * g + 1], c[4 * g + 2], c[4 * g + 3]), n * (MF::REGS / 4) + g);
          } else {
#pragma unroll
            for (int r = 0; r < 4; r++)
              if (col + r < N) epi.put1(erow + col + r, c[4 * g + r]);
          }
        }
    }
  } else {
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int r = 0; r < MF::REGS; r++) {
        const int rho = 8 * (r / 4) + q4 + r % 4;
        const int row = m0 + wm * WTM + (AK ? i * MS + rho : TM * rho + i);
        if (row >= M) continue;
        const uint64_t erow = (uint64_t)row * N;
        const int col = n0 + wn * WTN + TN * li;
        if (TN > 1 && vec_out && col + TN <= N) {
          if constexpr (TN == 4) epi.put4(erow + col, make_float4(acc[i][0][r], acc[i][1][r], acc[i][2][r], acc[i][3][r]), 0);
          else if constexpr (TN == 2) epi.put2(erow + col, make_float2(acc[i][0][r], acc[i][1][r]));
        } else {
#pragma unroll
          for (int n = 0; n < TN; n++)
            if (col + n < N) epi.put1(erow + col + n, acc[i][n][r]);
        }
      }
  }
}

// One product over the whole grid, with its own LDS.
template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, int MODE, int MS, class Epi>
__device__ __forceinline__ void gemm_mfma_block(const float* __restrict__ A, const float* __restrict__ B, int M, int N, int K,
                                                const int64_t* a_off, const int64_t* b_off, uint64_t a_stride, uint64_t b_stride, int splits,
                                                int k_per_split, const float* __restrict__ bias, uint32_t tiles_m, uint32_t tiles_n,
                                                int swizzle, Epi& epi) {
  __shared__ float smem[TileLds<BM, BN, BK, TA, TB>::FLOATS];
  gemm_mfma_tile<BM, BN, BK, WM, WN, TA, TB, MODE, MS>(A, B, M, N, K, a_off, b_off, a_stride, b_stride, splits, k_per_split, bias, tiles_m,
                                                      tiles_n, swizzle, epi, blockIdx.x, gridDim.x, smem);
}

}  // namespace rgg
