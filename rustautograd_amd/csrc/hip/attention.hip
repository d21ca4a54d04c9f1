// Fused scaled-dot-product attention, forward and backward, for the subgraph the planner matches:
//
//   S = q k^T;  Y = where(mask, S / c, fill);  P = exp(Y - max(Y)) / sum(exp(Y - max(Y)));  O = P v
//
// with its reverse-mode form (dv = P^T dO; dS = where(mask, P (dP - rowsum(P dP)), 0) / c with
// dP = dO v^T; dq = dS k; dk = dS^T q). The unfused graph materializes S, P and their gradients as
// [batch, heads, T, T] tensors; here they live in registers, 16x16 tiles at a time, and only q, k,
// v, O, their gradients and three per-row statistics touch HBM.
//
// Operands are strided views (AttnOperand): row t of problem b * heads + h starts at
// p + b sb + h sh + t st, so q, k and v are read straight out of the projection that produced them
// and O, dq, dk, dv are written into the layouts their readers use.
//
// A block runs 4, 8 or 16 wave64s (waves_for); each wave owns 16 rows (queries in the forward and
// the dq pass, keys in the dk/dv pass) and walks the other side in tiles of 16 with
// v_mfma_f32_16x16x4f32. A score tile is formed either as S^T (K supplies the MFMA rows) so that
// a lane holds four consecutive keys of one query, or as S (Q supplies the rows) so that a lane
// holds four consecutive queries of one key; either way the probabilities can feed the next
// product straight from registers, because within a group of 16 the lane's four k indices
// 4 (l / 16) + j are the same in both operands of a k-permuted MFMA sequence.
//
// The softmax runs in base 2 with the score scale folded into one operand: the kernels form
// S' = (q k^T) log2(e) / c by scaling q (or k) once, then P = exp2(Y' - max Y') / sum, with
// v_exp_f32 and a multiplication by the reciprocal row sum (in the forward, applied to each row
// of O = exp2(...) v rather than to every probability). This reassociates the graph's
// per-element divisions and exp by rounding-level amounts (1e-6 relative at most on P), the same
// order as the MFMA's own reduction differences, well inside the products' 1e-4 tolerance. The
// forward keeps a whole row of scores in registers (keys <= 256), so P comes from the final max
// and sum, as the backward recomputes it; the backward uses rowsum(P dP) = rowsum(dO * O), and
// its tile loops keep the next tile's score products in flight on the matrix cores while the
// vector units finish the current tile.
//
// Causal-style masks: the forward skips 16x16 tiles whose mask entries are all zero; the backward
// walks only the tiles between the first and the last key (or query) any row of the wave can
// see. Both are exact when every row has some visible key: the skipped probabilities underflow
// to exactly zero (exp(fill - max) with fill = -1e9), and hidden tiles inside the range
// contribute exact zeros. Waves with a fully masked row skip nothing.
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "ops.h"

namespace rgk {

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma4(floatx4 acc, float4 a, float4 b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, acc, 0, 0, 0);
  return acc;
}

// Lanes l, l ^ 16, l ^ 32, l ^ 48 share a row: combined by the permlane swaps (no LDS), every
// lane taking its two values in the same order.
__device__ __forceinline__ float row_max(float x) {
  float a, b;
  rg_swap16(x, &a, &b);
  rg_swap32(fmaxf(a, b), &a, &b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float row_sum(float x) {
  float a, b;
  rg_swap16(x, &a, &b);
  rg_swap32(a + b, &a, &b);
  return a + b;
}

constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// Packed mask tables of one (batch, head) slice, `words` 32-bit words each (attention_mask_words):
// row bits [tq][tk / 32] (bit j of word w: mask[q][32 w + j] != 0), column bits [tk][tq / 32]
// (bit j of word w: mask[32 w + j][k] != 0) and a visible flag per query row [tq].
struct MaskTables {
  const uint32_t *rows, *cols, *vis;
};

__device__ __forceinline__ uint32_t mask_slice(const AttnArgs& a, uint32_t bh) {
  const uint32_t b = bh / a.heads, h = bh % a.heads;
  return (a.mask_strides[0] ? b : 0) * (a.mask_strides[1] ? a.heads : 1) + (a.mask_strides[1] ? h : 0);
}

__device__ __forceinline__ uint64_t slice_words(int tq, int tk) { return 2 * (uint64_t)tq * tk / 32 + tq; }

__device__ __forceinline__ MaskTables mask_tables(const AttnArgs& a, uint32_t bh) {
  const uint32_t* base = a.mask_bits + mask_slice(a, bh) * slice_words(a.tq, a.tk);
  const uint64_t n = (uint64_t)a.tq * a.tk / 32;
  return {base, base + n, base + 2 * n};
}

constexpr uint64_t ALL_LANES = ~0ull;

// Row t of problem bh of an operand.
__device__ __forceinline__ const float* row_of(const AttnOperand& x, const AttnArgs& a, uint32_t bh, int t) {
  return x.p + (int64_t)(bh / a.heads) * x.sb + (int64_t)(bh % a.heads) * x.sh + (int64_t)t * x.st;
}
__device__ __forceinline__ float* out_row(const AttnOperand& x, const AttnArgs& a, uint32_t bh, int t) {
  return const_cast<float*>(row_of(x, a, bh, t));
}

// Builds the packed mask tables: one wave per query row (its row bits and visible flag) or per key
// column (its column bits) of one mask slice, 64 mask entries per ballot.
__global__ void __launch_bounds__(256) k_attn_mask_bits(AttnArgs a, uint32_t slices_h, uint32_t n_waves) {
  const uint32_t wv = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (wv >= n_waves) return;
  const int tq = a.tq, tk = a.tk;
  const uint32_t per = (uint32_t)(tq + tk), slice = wv / per, t = wv % per;
  const uint32_t b = slice / slices_h, h = slice % slices_h;
  const float* m = a.mask + (int64_t)b * a.mask_strides[0] + (int64_t)h * a.mask_strides[1];
  const int64_t sq = a.mask_strides[2], sk = a.mask_strides[3];
  const uint64_t n = (uint64_t)tq * tk / 32;
  uint32_t* base = a.mask_bits + (uint64_t)slice * (2 * n + tq);
  if (t < (uint32_t)tq) {  // row t: bits over keys, and whether any is set
    uint64_t any = 0;
    for (int c = 0; c < tk; c += 64) {
      const uint64_t bits = __ballot(c + (int)lane < tk && m[(int64_t)t * sq + (int64_t)(c + lane) * sk] != 0.0f);
      any |= bits;
      if (lane < 2 && c + 32 * (int)lane < tk) base[(uint64_t)t * (tk / 32) + c / 32 + lane] = (uint32_t)(bits >> (32 * lane));
    }
    if (lane == 0) base[2 * n + t] = any != 0;
  } else {  // column k: bits over queries
    const int k = (int)(t - tq);
    for (int c = 0; c < tq; c += 64) {
      const uint64_t bits = __ballot(c + (int)lane < tq && m[(int64_t)(c + lane) * sq + (int64_t)k * sk] != 0.0f);
      if (lane < 2 && c + 32 * (int)lane < tq) base[n + (uint64_t)k * (tq / 32) + c / 32 + lane] = (uint32_t)(bits >> (32 * lane));
    }
  }
}

__device__ __forceinline__ int wave_min(int x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = min(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ int wave_max(int x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = max(x, __shfl_xor(x, o));
  return x;
}

// Tiles [lo, hi) of 16 holding every set bit of each lane's bit row (`nw` words): the first and
// last set bits over the wave. With `skip` false (a row of the wave sees nothing, so its masked
// entries are not exactly zero), every tile.
__device__ __forceinline__ void tile_range(const uint32_t* words, int nw, bool skip, int n_tiles, int* lo, int* hi) {
  *lo = 0;
  *hi = n_tiles;
  if (!skip) return;
  int first = 1 << 30, last = -1;
  for (int i = 0; i < nw; i++) {
    const uint32_t w = words[i];
    if (w) {
      if (first == 1 << 30) first = 32 * i + __builtin_ctz(w);
      last = 32 * i + 31 - __builtin_clz(w);
    }
  }
  first = wave_min(first);
  last = wave_max(last);
  if (last < 0) {
    *hi = 0;
    return;
  }
  *lo = first / 16;
  *hi = last / 16 + 1;
}

// The 16-row tile of wave w. With 16 waves a block covers a whole 256-row problem, and under a
// causal mask the work of a tile grows with its index; waves are dealt to the four SIMDs in
// turn, so SIMD s gets tiles s, 7 - s, 8 + s and 15 - s: equal work on every SIMD.
template <int WAVES>
__device__ __forceinline__ int wave_tile(int w) {
  if constexpr (WAVES == 16) {
    const int j = w >> 2, s = w & 3;
    return j == 0 ? s : j == 1 ? 7 - s : j == 2 ? 8 + s : 15 - s;
  } else {
    return w;
  }
}

// Forward: one block per 16 * WAVES queries of one (batch, head); wave w owns queries
// q0 .. q0 + 15. Writes O and, per query, the row max (of the base-2 scores) and the row sum.
template <int HD, int NKT, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) k_attn_fwd(AttnArgs a) {
  constexpr int KP = HD + 4, TKP = NKT * 16 + 4, ND = HD / 16, NT = 64 * WAVES;
  __shared__ float Ks[NKT * 16 * KP];
  __shared__ float Vt[HD * TKP];
  const uint32_t bh = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int tq = a.tq, tk = a.tk, nkt = tk / 16;
  const float* Kb = row_of(a.k, a, bh, 0);
  const float* Vb = row_of(a.v, a, bh, 0);
  for (int i = tid; i < tk * HD / 4; i += NT) {
    const int key = i / (HD / 4), d = (i % (HD / 4)) * 4;
    *(float4*)&Ks[key * KP + d] = *(const float4*)(Kb + key * a.k.st + d);
    const float4 v = *(const float4*)(Vb + key * a.v.st + d);
    Vt[(d + 0) * TKP + key] = v.x;
    Vt[(d + 1) * TKP + key] = v.y;
    Vt[(d + 2) * TKP + key] = v.z;
    Vt[(d + 3) * TKP + key] = v.w;
  }
  __syncthreads();
  const int q0 = blockIdx.x * 16 * WAVES + wave_tile<WAVES>(w) * 16;
  if (q0 >= tq) return;
  const int l16 = lane & 15, g4 = (lane >> 4) * 4;
  const int q = q0 + l16;  // the lane's query in score tiles
  const float sc = LOG2E / a.div, fill = a.fill * LOG2E;
  float4 qf[ND];
#pragma unroll
  for (int n = 0; n < ND; n++) {
    const float4 x = *(const float4*)(row_of(a.q, a, bh, q) + n * 16 + g4);
    qf[n] = make_float4(x.x * sc, x.y * sc, x.z * sc, x.w * sc);
  }

  // Mask bits of the lane's four keys per tile; tiles with no visible key are skipped when every
  // row of the wave has a visible key.
  uint32_t bits[NKT];
  bool row_vis = true;
  if (a.mask_bits) {
    const MaskTables mt = mask_tables(a, bh);
    const uint32_t* mr = mt.rows + (uint64_t)q * (tk / 32);
    uint32_t any = 0;
#pragma unroll
    for (int kt = 0; kt < NKT; kt += 2) {
      const uint32_t word = kt < nkt ? mr[kt / 2] : 0u;
      any |= word;
      bits[kt] = word >> g4 & 0xF;
      bits[kt + 1] = word >> (16 + g4) & 0xF;
    }
    row_vis = any != 0;
  } else {
#pragma unroll
    for (int kt = 0; kt < NKT; kt++) bits[kt] = 0xF;
  }
  const bool all_vis = __ballot(row_vis) == ALL_LANES;
  uint32_t live = 0;  // bit kt: tile computed
#pragma unroll
  for (int kt = 0; kt < NKT; kt++)
    if (kt < nkt && (!all_vis || __ballot(bits[kt] != 0) != 0)) live |= 1u << kt;

  // Tiles every lane of the wave sees in full need no masking (all but the diagonal of a causal
  // mask).
  uint32_t full = 0;
#pragma unroll
  for (int kt = 0; kt < NKT; kt++)
    if (__ballot(bits[kt] != 0xF) == 0) full |= 1u << kt;

  // Scores, masked, and the row max; tiles in pairs for two independent MFMA chains.
  float s[NKT][4];
  float mx = -__builtin_huge_valf();
#pragma unroll
  for (int kt = 0; kt < NKT; kt += 2) {
    if (!(live >> kt & 3)) continue;
    floatx4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < ND; n++) {
      const float4 k0 = *(const float4*)&Ks[(kt * 16 + l16) * KP + n * 16 + g4];
      const float4 k1 = *(const float4*)&Ks[((kt + 1) * 16 + l16) * KP + n * 16 + g4];
      acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(k0.x, qf[n].x, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(k1.x, qf[n].x, acc1, 0, 0, 0);
      acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(k0.y, qf[n].y, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(k1.y, qf[n].y, acc1, 0, 0, 0);
      acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(k0.z, qf[n].z, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(k1.z, qf[n].z, acc1, 0, 0, 0);
      acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(k0.w, qf[n].w, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(k1.w, qf[n].w, acc1, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      s[kt][r] = (full >> kt & 1) || (bits[kt] >> r & 1) ? acc0[r] : fill;
      s[kt + 1][r] = (full >> (kt + 1) & 1) || (bits[kt + 1] >> r & 1) ? acc1[r] : fill;
    }
    // The max of each tile's four scores first, then one step into the running max.
    if (live >> kt & 1) mx = fmaxf(mx, fmaxf(fmaxf(s[kt][0], s[kt][1]), fmaxf(s[kt][2], s[kt][3])));
    if (live >> (kt + 1) & 1) mx = fmaxf(mx, fmaxf(fmaxf(s[kt + 1][0], s[kt + 1][1]), fmaxf(s[kt + 1][2], s[kt + 1][3])));
  }
  mx = row_max(mx);
  float z = 0.0f;
#pragma unroll
  for (int kt = 0; kt < NKT; kt++) {
    if (!(live >> kt & 1)) continue;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float e = exp2_hw(s[kt][r] - mx);
      s[kt][r] = e;
      z += e;
    }
  }
  z = row_sum(z);
  if (g4 == 0) {
    const uint64_t row = (uint64_t)bh * tq + q;
    a.stat_m[row] = mx;
    a.stat_z[row] = z;
  }
  // O = P V with P = e / z: the exponentials from registers (A operand: query l16, keys g4 + j),
  // V^T rows from LDS, and the division by the row sum applied once to each output; even and odd
  // tiles accumulate separately (independent MFMA chains) and are added at the end.
  floatx4 oacc[2][ND];
#pragma unroll
  for (int n = 0; n < ND; n++) oacc[0][n] = oacc[1][n] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kt = 0; kt < NKT; kt++) {
    if (!(live >> kt & 1)) continue;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int n = 0; n < ND; n++)
        oacc[kt & 1][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(s[kt][j], Vt[(n * 16 + l16) * TKP + kt * 16 + g4 + j], oacc[kt & 1][n], 0, 0, 0);
  }
  // Output row g4 + r belongs to query q0 + g4 + r, whose row sum lanes with l16 = g4 + r hold.
  float rzr[4];
#pragma unroll
  for (int r = 0; r < 4; r++) rzr[r] = 1.0f / __shfl(z, g4 + r);
#pragma unroll
  for (int r = 0; r < 4; r++) {
    float* orow = out_row(a.o, a, bh, q0 + g4 + r);
#pragma unroll
    for (int n = 0; n < ND; n++) orow[n * 16 + l16] = (oacc[0][n][r] + oacc[1][n][r]) * rzr[r];
  }
}

// Backward, query side: one block per 16 * WAVES queries; dq = dS k, and rowsum(dO * O) per
// query. The next key tile's scores and dP are in flight while the current tile's dS is formed
// and multiplied into dq.
template <int HD>
struct BwdQLds {
  static constexpr int KP = HD + 4;
  static constexpr int FLOATS = 2 * ATTN_MAX_KEYS * KP;  // K and V rows
};

// Block `bx` of problem `bh`, its K and V staged in `smem` (BwdQLds<HD>::FLOATS floats of LDS).
template <int HD, int WAVES>
__device__ __forceinline__ void bwd_q_block(const AttnArgs& a, uint32_t bx, uint32_t bh, float* smem) {
  constexpr int KP = HD + 4, ND = HD / 16, NT = 64 * WAVES;
  float* Ks = smem;
  float* Vs = smem + ATTN_MAX_KEYS * KP;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int tq = a.tq, tk = a.tk, nkt = tk / 16;
  const float* Kb = row_of(a.k, a, bh, 0);
  const float* Vb = row_of(a.v, a, bh, 0);
  for (int i = tid; i < tk * HD / 4; i += NT) {
    const int key = i / (HD / 4), d = (i % (HD / 4)) * 4;
    *(float4*)&Ks[key * KP + d] = *(const float4*)(Kb + key * a.k.st + d);
    *(float4*)&Vs[key * KP + d] = *(const float4*)(Vb + key * a.v.st + d);
  }
  __syncthreads();
  const int q0 = bx * 16 * WAVES + wave_tile<WAVES>(w) * 16;
  if (q0 >= tq) return;
  const int l16 = lane & 15, g4 = (lane >> 4) * 4;
  const int q = q0 + l16;
  const float *qrow = row_of(a.q, a, bh, q), *grow = row_of(a.d_o, a, bh, q), *orow = row_of(a.o_in, a, bh, q);
  const float sc = LOG2E / a.div, fill = a.fill * LOG2E, rdiv = 1.0f / a.div;
  float4 qf[ND], gf[ND];
  float dd = 0.0f;
#pragma unroll
  for (int n = 0; n < ND; n++) {
    const float4 x = *(const float4*)(qrow + n * 16 + g4);
    qf[n] = make_float4(x.x * sc, x.y * sc, x.z * sc, x.w * sc);
    gf[n] = *(const float4*)(grow + n * 16 + g4);
    const float4 o = *(const float4*)(orow + n * 16 + g4);
    dd += gf[n].x * o.x + gf[n].y * o.y + gf[n].z * o.z + gf[n].w * o.w;
  }
  dd = row_sum(dd);
  const uint64_t row = (uint64_t)bh * tq + q;
  const float mx = a.stat_m[row], rz = 1.0f / a.stat_z[row];
  if (g4 == 0) a.stat_dd[row] = dd;
  const uint32_t* mr = nullptr;
  bool row_vis = true;
  if (a.mask_bits) {
    const MaskTables mt = mask_tables(a, bh);
    mr = mt.rows + (uint64_t)q * (tk / 32);
    row_vis = mt.vis[q] != 0;
  }
  int lo = 0, hi = nkt;
  if (mr) tile_range(mr, tk / 32, __ballot(row_vis) == ALL_LANES, nkt, &lo, &hi);
  auto scores = [&](int kt, floatx4& sacc, floatx4& pacc) {
    sacc = pacc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < ND; n++) {
      const float4 kk = *(const float4*)&Ks[(kt * 16 + l16) * KP + n * 16 + g4];
      const float4 vv = *(const float4*)&Vs[(kt * 16 + l16) * KP + n * 16 + g4];
      sacc = mfma4(sacc, kk, qf[n]);
      pacc = mfma4(pacc, vv, gf[n]);
    }
  };
  floatx4 dacc[ND];
#pragma unroll
  for (int n = 0; n < ND; n++) dacc[n] = floatx4{0.f, 0.f, 0.f, 0.f};
  floatx4 s_cur = {0.f, 0.f, 0.f, 0.f}, p_cur = s_cur;
  if (lo < hi) scores(lo, s_cur, p_cur);
  for (int kt = lo; kt < hi; kt++) {
    floatx4 s_nxt = s_cur, p_nxt = p_cur;
    if (kt + 1 < hi) scores(kt + 1, s_nxt, p_nxt);
    // s_cur[r] = S'[q][key], p_cur[r] = dP[q][key] for key = kt * 16 + g4 + r.
    const uint32_t bits = mr ? (mr[kt >> 1] >> (((kt & 1) << 4) + g4)) & 0xF : 0xF;
    float ds[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const bool vis = bits >> r & 1;
      const float p = exp2_hw((vis ? s_cur[r] : fill) - mx) * rz;
      ds[r] = vis ? p * (p_cur[r] - dd) * rdiv : 0.0f;
    }
    // dq += dS K: A = dS (query l16, keys g4 + j), B = K rows g4 + j of the tile, column n*16 + l16.
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int n = 0; n < ND; n++)
        dacc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(ds[j], Ks[(kt * 16 + g4 + j) * KP + n * 16 + l16], dacc[n], 0, 0, 0);
    s_cur = s_nxt;
    p_cur = p_nxt;
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    float* drow = out_row(a.dq, a, bh, q0 + g4 + r);
#pragma unroll
    for (int n = 0; n < ND; n++) drow[n * 16 + l16] = dacc[n][r];
  }
  if (a.colp) {
    // dq's column sums over the problem's rows (every wave holds 16 of them): each lane's four
    // rows in order, the wave's four row groups by a fixed butterfly, then the waves in order
    // through LDS (the K rows' space, every wave past its products).
    float cs[ND];
#pragma unroll
    for (int n = 0; n < ND; n++) {
      cs[n] = ((dacc[n][0] + dacc[n][1]) + dacc[n][2]) + dacc[n][3];
      cs[n] = cs[n] + __shfl_xor(cs[n], 16);
      cs[n] = cs[n] + __shfl_xor(cs[n], 32);
    }
    __syncthreads();
    if (lane < 16)
#pragma unroll
      for (int n = 0; n < ND; n++) Ks[w * HD + n * 16 + l16] = cs[n];
    __syncthreads();
    if (tid < HD) {
      float t = Ks[tid];
      for (int q = 1; q < WAVES; q++) t = t + Ks[q * HD + tid];
      a.colp[(uint64_t)(bh / a.heads) * a.col_len + a.col_q + (bh % a.heads) * a.dq.sh + tid] = t;
    }
  }
}

// Backward, key side: one block per 16 * WAVES keys; dv = P^T dO and dk = dS^T q over the query
// tiles that see the wave's keys. The tile loop has scalar control and a body without branches or
// global memory access (the mask words sit in LDS): the next tile's scores, dP and mask word are
// in flight while the current tile is consumed. (Measured on C4's shapes: 7 % faster than a loop
// with a conditional next-tile block and the mask word picked from registers by a select chain.)
template <int HD, int WAVES>
struct BwdKvLds {
  static constexpr int KP = HD + 4, NW = ATTN_MAX_KEYS / 32;
  static constexpr bool MW_LDS = HD <= 32;  // mask words in LDS where they fit beside the operand tiles
  static constexpr int ROWS = 2 * ATTN_MAX_KEYS * KP;  // q and dO rows
  // Then per query a float4 (row max, 1 / row sum, rowsum(dO * O)) and the mask words.
  static constexpr int FLOATS = ROWS + 4 * ATTN_MAX_KEYS + (MW_LDS ? WAVES * NW * 64 : 1);
};

// Block `bx` of problem `bh`, its q, dO, statistics and mask words staged in `smem`
// (BwdKvLds<HD, WAVES>::FLOATS floats of LDS, 16-byte aligned).
template <int HD, int WAVES>
__device__ __forceinline__ void bwd_kv_block(const AttnArgs& a, uint32_t bx, uint32_t bh, float* smem) {
  constexpr int KP = HD + 4, ND = HD / 16, NT = 64 * WAVES, NW = ATTN_MAX_KEYS / 32;
  typedef BwdKvLds<HD, WAVES> L;
  float* Qs = smem;
  float* Gs = smem + ATTN_MAX_KEYS * KP;
  // Per query: row max, 1 / row sum, rowsum(dO * O). (Folding log2 of the sum into the max would
  // lose it next to the fill value's max of a fully masked row.)
  float4* St = (float4*)(smem + L::ROWS);
  constexpr bool MW_LDS = L::MW_LDS;
  uint32_t* Mw = (uint32_t*)(smem + L::ROWS + 4 * ATTN_MAX_KEYS);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int tq = a.tq, tk = a.tk, nqt = tq / 16;
  const int k0 = bx * 16 * WAVES + wave_tile<WAVES>(w) * 16;
  const bool active = k0 < tk;
  const int l16 = lane & 15, g4 = (lane >> 4) * 4;
  const int key = k0 + l16;  // the lane's key in score tiles
  MaskTables mt{nullptr, nullptr, nullptr};
  if (a.mask_bits) mt = mask_tables(a, bh);
  const float* Qb = row_of(a.q, a, bh, 0);
  const float* Gb = row_of(a.d_o, a, bh, 0);
  for (int i = tid; i < tq * HD / 4; i += NT) {
    const int qq = i / (HD / 4), d = (i % (HD / 4)) * 4;
    *(float4*)&Qs[qq * KP + d] = *(const float4*)(Qb + qq * a.q.st + d);
    *(float4*)&Gs[qq * KP + d] = *(const float4*)(Gb + qq * a.d_o.st + d);
  }
  const uint64_t srow = (uint64_t)bh * tq;
  int vis_all = 1;
  for (int i = tid; i < tq; i += NT) {
    St[i] = make_float4(a.stat_m[srow + i], 1.0f / a.stat_z[srow + i], a.stat_dd[srow + i], 0.0f);
    if (mt.vis && !mt.vis[i]) vis_all = 0;
  }
  // Every query row sees some key: then masked entries are exactly zero and may be skipped.
  const bool all_vis = __syncthreads_and(vis_all);
  if (!active) return;
  // The wave's own keys: k (scaled) and v rows, and the key's mask column, 32 queries per word.
  // (Loading them before the staging loop measured slower: they delay the staged tiles every
  // wave waits for.)
  const float sc = LOG2E / a.div, fill = a.fill * LOG2E, rdiv = 1.0f / a.div;
  float4 kf[ND], vf[ND];
#pragma unroll
  for (int n = 0; n < ND; n++) {
    const float4 x = *(const float4*)(row_of(a.k, a, bh, key) + n * 16 + g4);
    kf[n] = make_float4(x.x * sc, x.y * sc, x.z * sc, x.w * sc);
    vf[n] = *(const float4*)(row_of(a.v, a, bh, key) + n * 16 + g4);
  }
  uint32_t cb[NW];
#pragma unroll
  for (int i = 0; i < NW; i++) cb[i] = (mt.cols && i < tq / 32) ? mt.cols[(uint64_t)key * (tq / 32) + i] : ~0u;
  int lo = 0, hi = nqt;
  if (mt.cols) tile_range(cb, tq / 32, all_vis, nqt, &lo, &hi);
  // The range is the same in every lane: scalar loop control.
  lo = __builtin_amdgcn_readfirstlane(lo);
  hi = __builtin_amdgcn_readfirstlane(hi);
  auto scores = [&](int qt, floatx4& sacc, floatx4& pacc) {
    sacc = pacc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < ND; n++) {
      const float4 qq = *(const float4*)&Qs[(qt * 16 + l16) * KP + n * 16 + g4];
      const float4 gg = *(const float4*)&Gs[(qt * 16 + l16) * KP + n * 16 + g4];
      sacc = mfma4(sacc, qq, kf[n]);
      pacc = mfma4(pacc, gg, vf[n]);
    }
  };
  // The lane's mask column in LDS, word-major, so that the tile loop reads word qt / 2 with one
  // conflict-free access (a register array indexed by the tile would go to scratch memory).
  uint32_t* mw = Mw + (MW_LDS ? w * NW * 64 + lane : 0);
  if constexpr (MW_LDS) {
#pragma unroll
    for (int i = 0; i < NW; i++) mw[i * 64] = cb[i];
  }
  auto mask_word = [&](int qt) -> uint32_t {
    if constexpr (MW_LDS) return mw[(qt >> 1) * 64];
    else return mt.cols ? mt.cols[(uint64_t)key * (tq / 32) + (qt >> 1)] : ~0u;
  };
  floatx4 kacc[ND], vacc[ND];
#pragma unroll
  for (int n = 0; n < ND; n++) kacc[n] = vacc[n] = floatx4{0.f, 0.f, 0.f, 0.f};
  // Tile qt from its scores s[r] = S'[qb + r][key] and dP p[r] = dP[qb + r][key] for the lane's
  // queries qb = qt * 16 + g4.
  auto consume = [&](int qt, const floatx4& s, const floatx4& pp, uint32_t word) {
    // B operands of dv += P^T dO and dk += dS^T q (rows g4 + j of the tile, column n * 16 + l16),
    // and the statistics of the lane's four queries.
    float gb[4][ND], qb[4][ND];
    float4 st[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      st[j] = St[qt * 16 + g4 + j];
#pragma unroll
      for (int n = 0; n < ND; n++) {
        gb[j][n] = Gs[(qt * 16 + g4 + j) * KP + n * 16 + l16];
        qb[j][n] = Qs[(qt * 16 + g4 + j) * KP + n * 16 + l16];
      }
    }
    const uint32_t bits = word >> (((qt & 1) << 4) + g4) & 0xF;
    float p[4], ds[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const bool vis = bits >> r & 1;
      p[r] = exp2_hw((vis ? s[r] : fill) - st[r].x) * st[r].y;
      ds[r] = vis ? p[r] * (pp[r] - st[r].z) : 0.0f;
    }
    // A = P^T / (dS c)^T (key l16, queries g4 + j); dk's 1 / c is applied to the finished sums.
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int n = 0; n < ND; n++) {
        vacc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[j], gb[j][n], vacc[n], 0, 0, 0);
        kacc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(ds[j], qb[j][n], kacc[n], 0, 0, 0);
      }
  };
  // The last tile is consumed after the loop, so that the loop body needs no branch.
  floatx4 s_cur = {0.f, 0.f, 0.f, 0.f}, p_cur = s_cur;
  uint32_t w_cur = ~0u;
  if (lo < hi) {
    scores(lo, s_cur, p_cur);
    w_cur = mask_word(lo);
  }
  for (int qt = lo; qt + 1 < hi; qt++) {
    floatx4 s_nxt, p_nxt;
    const uint32_t w_nxt = mask_word(qt + 1);
    scores(qt + 1, s_nxt, p_nxt);
    consume(qt, s_cur, p_cur, w_cur);
    s_cur = s_nxt;
    p_cur = p_nxt;
    w_cur = w_nxt;
  }
  if (lo < hi) consume(hi - 1, s_cur, p_cur, w_cur);
#pragma unroll
  for (int r = 0; r < 4; r++) {
    float* krow = out_row(a.dk, a, bh, k0 + g4 + r);
    float* vrow = out_row(a.dv, a, bh, k0 + g4 + r);
#pragma unroll
    for (int n = 0; n < ND; n++) {
      krow[n * 16 + l16] = kacc[n][r] * rdiv;
      vrow[n * 16 + l16] = vacc[n][r];
    }
  }
  if (a.colp) {
    // dk's and dv's column sums over the problem's rows, as the query pass sums dq's (through the
    // q rows' space): the stored values, each lane's four rows in order, a fixed butterfly over
    // the wave's row groups, the waves in order.
    float ck[ND], cv[ND];
#pragma unroll
    for (int n = 0; n < ND; n++) {
      ck[n] = ((kacc[n][0] * rdiv + kacc[n][1] * rdiv) + kacc[n][2] * rdiv) + kacc[n][3] * rdiv;
      cv[n] = ((vacc[n][0] + vacc[n][1]) + vacc[n][2]) + vacc[n][3];
      ck[n] = ck[n] + __shfl_xor(ck[n], 16);
      ck[n] = ck[n] + __shfl_xor(ck[n], 32);
      cv[n] = cv[n] + __shfl_xor(cv[n], 16);
      cv[n] = cv[n] + __shfl_xor(cv[n], 32);
    }
    __syncthreads();
    if (lane < 16)
#pragma unroll
      for (int n = 0; n < ND; n++) {
        Qs[w * 2 * HD + n * 16 + l16] = ck[n];
        Qs[w * 2 * HD + HD + n * 16 + l16] = cv[n];
      }
    __syncthreads();
    if (tid < 2 * HD) {
      float t = Qs[tid];
      for (int q = 1; q < WAVES; q++) t = t + Qs[q * 2 * HD + tid];
      const uint32_t h = bh % a.heads;
      const int64_t col = tid < HD ? a.col_k + h * a.dk.sh + tid : a.col_v + h * a.dv.sh + (tid - HD);
      a.colp[(uint64_t)(bh / a.heads) * a.col_len + col] = t;
    }
  }
}

template <int HD, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) k_attn_bwd_q(AttnArgs a) {
  __shared__ float4 smem[BwdQLds<HD>::FLOATS / 4];
  bwd_q_block<HD, WAVES>(a, blockIdx.x, blockIdx.y, (float*)smem);
}

template <int HD, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) k_attn_bwd_kv(AttnArgs a) {
  __shared__ float4 smem[(BwdKvLds<HD, WAVES>::FLOATS + 3) / 4];
  bwd_kv_block<HD, WAVES>(a, blockIdx.x, blockIdx.y, (float*)smem);
}

// Both backward passes in one launch: the problems' query-pass blocks at y < bh, their key-pass
// blocks after them, over one LDS buffer sized for the larger. Each block runs the code of its
// pass's own kernel: one launch instead of two, and the key pass's blocks start on the CUs the
// query pass's blocks leave.
template <int HD, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) k_attn_bwd(AttnArgs a) {
  constexpr int F = BwdKvLds<HD, WAVES>::FLOATS > BwdQLds<HD>::FLOATS ? BwdKvLds<HD, WAVES>::FLOATS : BwdQLds<HD>::FLOATS;
  __shared__ float4 smem[(F + 3) / 4];
  if (blockIdx.y < a.bh) bwd_q_block<HD, WAVES>(a, blockIdx.x, blockIdx.y, (float*)smem);
  else bwd_kv_block<HD, WAVES>(a, blockIdx.x, blockIdx.y - a.bh, (float*)smem);
}

// Sixteen waves (a whole 256-row problem per block: its K and V, or q and dO, are staged once)
// when there are problems for every CU; else four waves per block unless the launch would still
// give every CU two blocks with eight.
int waves_for(const AttnArgs& a, int rows) {
  if (rows == 256 && a.bh >= 256) return 16;
  return (uint64_t)a.bh * ((rows + 127) / 128) >= 512 ? 8 : 4;
}

template <int HD>
void forward_hd(hipStream_t s, const AttnArgs& a) {
  const int wv = waves_for(a, a.tq);
  const dim3 grid((uint32_t)((a.tq + 16 * wv - 1) / (16 * wv)), a.bh);
  if (wv == 16) hipLaunchKernelGGL((k_attn_fwd<HD, ATTN_MAX_KEYS / 16, 16>), grid, dim3(1024), 0, s, a);
  else if (wv == 8) hipLaunchKernelGGL((k_attn_fwd<HD, ATTN_MAX_KEYS / 16, 8>), grid, dim3(512), 0, s, a);
  else hipLaunchKernelGGL((k_attn_fwd<HD, ATTN_MAX_KEYS / 16, 4>), grid, dim3(256), 0, s, a);
}

template <int HD>
void backward_hd(hipStream_t s, const AttnArgs& a) {
  // Equal grids (as many queries as keys, a whole problem per block): both passes in one launch.
  if (a.tq == a.tk && waves_for(a, a.tq) == 16) {
    const dim3 grid((uint32_t)((a.tq + 255) / 256), 2 * a.bh);
    hipLaunchKernelGGL((k_attn_bwd<HD, 16>), grid, dim3(1024), 0, s, a);
    return;
  }
  {
    const int wv = waves_for(a, a.tq);
    const dim3 grid((uint32_t)((a.tq + 16 * wv - 1) / (16 * wv)), a.bh);
    if (wv == 16) hipLaunchKernelGGL((k_attn_bwd_q<HD, 16>), grid, dim3(1024), 0, s, a);
    else if (wv == 8) hipLaunchKernelGGL((k_attn_bwd_q<HD, 8>), grid, dim3(512), 0, s, a);
    else hipLaunchKernelGGL((k_attn_bwd_q<HD, 4>), grid, dim3(256), 0, s, a);
  }
  {
    const int wv = waves_for(a, a.tk);
    const dim3 grid((uint32_t)((a.tk + 16 * wv - 1) / (16 * wv)), a.bh);
    if (wv == 16) hipLaunchKernelGGL((k_attn_bwd_kv<HD, 16>), grid, dim3(1024), 0, s, a);
    else if (wv == 8) hipLaunchKernelGGL((k_attn_bwd_kv<HD, 8>), grid, dim3(512), 0, s, a);
    else hipLaunchKernelGGL((k_attn_bwd_kv<HD, 4>), grid, dim3(256), 0, s, a);
  }
}

}  // namespace

bool attention_supported(int dtype, int64_t hd, int64_t tq, int64_t tk) {
  return dtype == RG_F32 && (hd == 16 || hd == 32 || hd == 64) && tq > 0 && tk > 0 && tq % 32 == 0 && tk % 32 == 0 &&
         tk <= ATTN_MAX_KEYS && tq <= ATTN_MAX_KEYS;
}

uint64_t attention_mask_words(const AttnArgs& a) {
  if (!a.mask) return 0;
  const uint64_t slices = (a.mask_strides[0] ? a.bh / a.heads : 1) * (a.mask_strides[1] ? a.heads : 1);
  return slices * (2 * (uint64_t)a.tq * a.tk / 32 + a.tq);
}

void attention_forward(hipStream_t s, const AttnArgs& a, bool build_mask_bits) {
  if (a.mask && build_mask_bits) {
    const uint64_t slices = (a.mask_strides[0] ? a.bh / a.heads : 1) * (a.mask_strides[1] ? a.heads : 1);
    const uint32_t waves = (uint32_t)(slices * (uint64_t)(a.tq + a.tk));
    hipLaunchKernelGGL(k_attn_mask_bits, dim3((waves + 3) / 4), dim3(256), 0, s, a, a.mask_strides[1] ? a.heads : 1u, waves);
  }
  if (a.hd == 16) forward_hd<16>(s, a);
  else if (a.hd == 32) forward_hd<32>(s, a);
  else forward_hd<64>(s, a);
}

bool attention_backward_column_sums(const AttnArgs& a) {
  return a.tq == a.tk && a.tq == 256 && a.bh >= 256 && a.bh % a.heads == 0;
}

void attention_backward(hipStream_t s, const AttnArgs& a) {
  if (a.colp && !attention_backward_column_sums(a)) throw std::runtime_error("attention backward: column sums for these shapes");
  if (a.hd == 16) backward_hd<16>(s, a);
  else if (a.hd == 32) backward_hd<32>(s, a);
  else backward_hd<64>(s, a);
}

}  // namespace rgk
