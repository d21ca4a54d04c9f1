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
// Every kernel runs four wave64s per block; each wave owns 16 rows (queries in the forward and
// the dq pass, keys in the dk/dv pass) and walks the other side in tiles of 16 with
// v_mfma_f32_16x16x4f32. A score tile is formed either as S^T (K supplies the MFMA rows) so that
// a lane holds four consecutive keys of one query, or as S (Q supplies the rows) so that a lane
// holds four consecutive queries of one key; either way the probabilities can feed the next
// product straight from registers, because within a group of 16 the lane's four k indices
// 4 (l / 16) + j are the same in both operands of a k-permuted MFMA sequence.
//
// The softmax runs in base 2 with the score scale folded into one operand: the kernels form
// S' = (q k^T) log2(e) / c by scaling q (or k) once, then P = exp2(Y' - max Y') / sum, with
// v_exp_f32 and a multiplication by the reciprocal row sum. This reassociates the graph's
// per-element divisions and exp by rounding-level amounts (1e-6 relative at most on P), the same
// order as the MFMA's own reduction differences, well inside the products' 1e-4 tolerance. The
// forward keeps a whole row of scores in registers (keys <= 256), so P comes from the final max
// and sum, not from online rescaling. The backward recomputes P from the saved max and sum and
// uses rowsum(P dP) = rowsum(dO * O).
//
// Causal-style masks: a 16x16 tile whose mask entries are all zero is skipped, which is exact
// when every row of the tile has some visible key: its probabilities underflow to exactly zero
// (exp(fill - max) with fill = -1e9). Waves with a fully masked row skip nothing.
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

// Lanes l, l ^ 16, l ^ 32, l ^ 48 share a row.
__device__ __forceinline__ float row_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float row_sum(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
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

// Builds the packed mask tables: one thread per word.
__global__ void __launch_bounds__(256) k_attn_mask_bits(AttnArgs a, uint32_t slices_h, uint64_t n_words) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n_words) return;
  const int tq = a.tq, tk = a.tk;
  const uint64_t per = slice_words(tq, tk), n = (uint64_t)tq * tk / 32;
  const uint32_t slice = (uint32_t)(i / per), b = slice / slices_h, h = slice % slices_h;
  const uint64_t t = i % per;
  const float* m = a.mask + (int64_t)b * a.mask_strides[0] + (int64_t)h * a.mask_strides[1];
  const int64_t sq = a.mask_strides[2], sk = a.mask_strides[3];
  uint32_t word = 0;
  if (t < n) {  // row bits
    const int q = (int)(t / (tk / 32)), w = (int)(t % (tk / 32));
    for (int j = 0; j < 32; j++) word |= (m[q * sq + (int64_t)(32 * w + j) * sk] != 0.0f ? 1u : 0u) << j;
  } else if (t < 2 * n) {  // column bits
    const int k = (int)((t - n) / (tq / 32)), w = (int)((t - n) % (tq / 32));
    for (int j = 0; j < 32; j++) word |= (m[(int64_t)(32 * w + j) * sq + k * sk] != 0.0f ? 1u : 0u) << j;
  } else {  // some key visible in row q
    const int q = (int)(t - 2 * n);
    for (int k = 0; k < tk && !word; k++) word = m[q * sq + k * sk] != 0.0f;
  }
  a.mask_bits[i] = word;
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
  const int q0 = blockIdx.x * 16 * WAVES + w * 16;
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
      const float y0 = (bits[kt] >> r & 1) ? acc0[r] : fill;
      const float y1 = (bits[kt + 1] >> r & 1) ? acc1[r] : fill;
      s[kt][r] = y0;
      s[kt + 1][r] = y1;
      if (live >> kt & 1) mx = fmaxf(mx, y0);
      if (live >> (kt + 1) & 1) mx = fmaxf(mx, y1);
    }
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
  // O = P V: P from registers (A operand: query l16, keys g4 + j), V^T rows from LDS; even and
  // odd tiles accumulate separately (independent MFMA chains) and are added at the end.
  const float rz = 1.0f / z;
  floatx4 oacc[2][ND];
#pragma unroll
  for (int n = 0; n < ND; n++) oacc[0][n] = oacc[1][n] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kt = 0; kt < NKT; kt++) {
    if (!(live >> kt & 1)) continue;
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; r++) p[r] = s[kt][r] * rz;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int n = 0; n < ND; n++)
        oacc[kt & 1][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[j], Vt[(n * 16 + l16) * TKP + kt * 16 + g4 + j], oacc[kt & 1][n], 0, 0, 0);
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    float* orow = out_row(a.o, a, bh, q0 + g4 + r);
#pragma unroll
    for (int n = 0; n < ND; n++) orow[n * 16 + l16] = oacc[0][n][r] + oacc[1][n][r];
  }
}

// Backward, query side: one block per 16 * WAVES queries; dq = dS k, and rowsum(dO * O) per query.
template <int HD, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) k_attn_bwd_q(AttnArgs a) {
  constexpr int KP = HD + 4, ND = HD / 16, NT = 64 * WAVES;
  __shared__ float Ks[ATTN_MAX_KEYS * KP];
  __shared__ float Vs[ATTN_MAX_KEYS * KP];
  const uint32_t bh = blockIdx.y;
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
  const int q0 = blockIdx.x * 16 * WAVES + w * 16;
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
  const float mx = a.stat_m[row], z = a.stat_z[row];
  if (g4 == 0) a.stat_dd[row] = dd;
  const uint32_t* mr = nullptr;
  bool row_vis = true;
  if (a.mask_bits) {
    const MaskTables mt = mask_tables(a, bh);
    mr = mt.rows + (uint64_t)q * (tk / 32);
    row_vis = mt.vis[q] != 0;
  }
  const bool all_vis = __ballot(row_vis) == ALL_LANES;
  const float rz = 1.0f / z;

  floatx4 dacc[2][ND];
#pragma unroll
  for (int n = 0; n < ND; n++) dacc[0][n] = dacc[1][n] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int kt = 0; kt < nkt; kt++) {
    uint32_t bits = 0xF;
    if (mr) {
      bits = mr[kt >> 1] >> (((kt & 1) << 4) + g4) & 0xF;
      if (all_vis && __ballot(bits != 0) == 0) continue;
    }
    floatx4 sacc = {0.f, 0.f, 0.f, 0.f}, pacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < ND; n++) {
      const float4 kk = *(const float4*)&Ks[(kt * 16 + l16) * KP + n * 16 + g4];
      const float4 vv = *(const float4*)&Vs[(kt * 16 + l16) * KP + n * 16 + g4];
      sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.x, qf[n].x, sacc, 0, 0, 0);
      pacc = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.x, gf[n].x, pacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.y, qf[n].y, sacc, 0, 0, 0);
      pacc = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.y, gf[n].y, pacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.z, qf[n].z, sacc, 0, 0, 0);
      pacc = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.z, gf[n].z, pacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.w, qf[n].w, sacc, 0, 0, 0);
      pacc = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.w, gf[n].w, pacc, 0, 0, 0);
    }
    // sacc[r] = S[q][key], pacc[r] = dP[q][key] for key = kt * 16 + g4 + r.
    float ds[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const bool vis = bits >> r & 1;
      const float p = exp2_hw((vis ? sacc[r] : fill) - mx) * rz;
      ds[r] = vis ? p * (pacc[r] - dd) * rdiv : 0.0f;
    }
    // dq += dS K: A = dS (query l16, keys g4 + j), B = K rows g4 + j of the tile, column n*16 + l16.
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int n = 0; n < ND; n++)
        dacc[kt & 1][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(ds[j], Ks[(kt * 16 + g4 + j) * KP + n * 16 + l16], dacc[kt & 1][n], 0, 0, 0);
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    float* drow = out_row(a.dq, a, bh, q0 + g4 + r);
#pragma unroll
    for (int n = 0; n < ND; n++) drow[n * 16 + l16] = dacc[0][n][r] + dacc[1][n][r];
  }
}

// Backward, key side: one block per 16 * WAVES keys; dv = P^T dO and dk = dS^T q over all queries.
template <int HD, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) k_attn_bwd_kv(AttnArgs a) {
  constexpr int KP = HD + 4, ND = HD / 16, NT = 64 * WAVES, NW = ATTN_MAX_KEYS / 32;
  __shared__ float Qs[ATTN_MAX_KEYS * KP];
  __shared__ float Gs[ATTN_MAX_KEYS * KP];
  __shared__ float4 St[ATTN_MAX_KEYS];  // per query: row max, row sum, rowsum(dO * O), 1 / row sum
  __shared__ uint32_t Rv[ATTN_MAX_KEYS];  // per query: some key visible
  const uint32_t bh = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int tq = a.tq, tk = a.tk, nqt = tq / 16;
  const float* Qb = row_of(a.q, a, bh, 0);
  const float* Gb = row_of(a.d_o, a, bh, 0);
  for (int i = tid; i < tq * HD / 4; i += NT) {
    const int qq = i / (HD / 4), d = (i % (HD / 4)) * 4;
    *(float4*)&Qs[qq * KP + d] = *(const float4*)(Qb + qq * a.q.st + d);
    *(float4*)&Gs[qq * KP + d] = *(const float4*)(Gb + qq * a.d_o.st + d);
  }
  const uint64_t srow = (uint64_t)bh * tq;
  MaskTables mt{nullptr, nullptr, nullptr};
  if (a.mask_bits) mt = mask_tables(a, bh);
  for (int i = tid; i < tq; i += NT) {
    const float zz = a.stat_z[srow + i];
    St[i] = make_float4(a.stat_m[srow + i], zz, a.stat_dd[srow + i], 1.0f / zz);
    Rv[i] = mt.vis ? mt.vis[i] : 1u;
  }
  __syncthreads();
  const int k0 = blockIdx.x * 16 * WAVES + w * 16;
  if (k0 >= tk) return;
  const int l16 = lane & 15, g4 = (lane >> 4) * 4;
  const int key = k0 + l16;  // the lane's key in score tiles
  const float sc = LOG2E / a.div, fill = a.fill * LOG2E, rdiv = 1.0f / a.div;
  float4 kf[ND], vf[ND];
#pragma unroll
  for (int n = 0; n < ND; n++) {
    const float4 x = *(const float4*)(row_of(a.k, a, bh, key) + n * 16 + g4);
    kf[n] = make_float4(x.x * sc, x.y * sc, x.z * sc, x.w * sc);
    vf[n] = *(const float4*)(row_of(a.v, a, bh, key) + n * 16 + g4);
  }
  // The lane's key column of the mask, 32 queries per word.
  uint32_t cb[NW];
#pragma unroll
  for (int i = 0; i < NW; i++) cb[i] = (mt.cols && i < tq / 32) ? mt.cols[(uint64_t)key * (tq / 32) + i] : ~0u;
  floatx4 kacc[2][ND], vacc[2][ND];
#pragma unroll
  for (int n = 0; n < ND; n++) kacc[0][n] = kacc[1][n] = vacc[0][n] = vacc[1][n] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int qt = 0; qt < nqt; qt++) {
    const int qb = qt * 16 + g4;  // the lane's four queries qb .. qb + 3
    uint32_t word = cb[0];
#pragma unroll
    for (int i = 1; i < NW; i++)
      if (qt >> 1 == i) word = cb[i];
    const uint32_t bits = word >> (((qt & 1) << 4) + g4) & 0xF;
    if (mt.cols) {
      const bool vis4 = Rv[qb] && Rv[qb + 1] && Rv[qb + 2] && Rv[qb + 3];
      if (__ballot(vis4) == ALL_LANES && __ballot(bits != 0) == 0) continue;
    }
    floatx4 sacc = {0.f, 0.f, 0.f, 0.f}, pacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < ND; n++) {
      const float4 qq = *(const float4*)&Qs[(qt * 16 + l16) * KP + n * 16 + g4];
      const float4 gg = *(const float4*)&Gs[(qt * 16 + l16) * KP + n * 16 + g4];
      sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qq.x, kf[n].x, sacc, 0, 0, 0);
      pacc = __builtin_amdgcn_mfma_f32_16x16x4f32(gg.x, vf[n].x, pacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qq.y, kf[n].y, sacc, 0, 0, 0);
      pacc = __builtin_amdgcn_mfma_f32_16x16x4f32(gg.y, vf[n].y, pacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qq.z, kf[n].z, sacc, 0, 0, 0);
      pacc = __builtin_amdgcn_mfma_f32_16x16x4f32(gg.z, vf[n].z, pacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qq.w, kf[n].w, sacc, 0, 0, 0);
      pacc = __builtin_amdgcn_mfma_f32_16x16x4f32(gg.w, vf[n].w, pacc, 0, 0, 0);
    }
    // sacc[r] = S[qb + r][key], pacc[r] = dP[qb + r][key].
    float p[4], ds[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const bool vis = bits >> r & 1;
      const float4 st = St[qb + r];
      p[r] = exp2_hw((vis ? sacc[r] : fill) - st.x) * st.w;
      ds[r] = vis ? p[r] * (pacc[r] - st.z) * rdiv : 0.0f;
    }
    // dv += P^T dO, dk += dS^T q: A = P^T / dS^T (key l16, queries g4 + j), B = rows g4 + j of the tile.
    floatx4* va = vacc[qt & 1];
    floatx4* ka = kacc[qt & 1];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int n = 0; n < ND; n++) {
        va[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[j], Gs[(qt * 16 + g4 + j) * KP + n * 16 + l16], va[n], 0, 0, 0);
        ka[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(ds[j], Qs[(qt * 16 + g4 + j) * KP + n * 16 + l16], ka[n], 0, 0, 0);
      }
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    float* krow = out_row(a.dk, a, bh, k0 + g4 + r);
    float* vrow = out_row(a.dv, a, bh, k0 + g4 + r);
#pragma unroll
    for (int n = 0; n < ND; n++) {
      krow[n * 16 + l16] = kacc[0][n][r] + kacc[1][n][r];
      vrow[n * 16 + l16] = vacc[0][n][r] + vacc[1][n][r];
    }
  }
}

// Four waves per block unless the launch would still give every CU two blocks with eight.
int waves_for(const AttnArgs& a, int rows) { return (uint64_t)a.bh * ((rows + 127) / 128) >= 512 ? 8 : 4; }

template <int HD>
void forward_hd(hipStream_t s, const AttnArgs& a) {
  if (waves_for(a, a.tq) == 8)
    hipLaunchKernelGGL((k_attn_fwd<HD, ATTN_MAX_KEYS / 16, 8>), dim3((uint32_t)((a.tq + 127) / 128), a.bh), dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL((k_attn_fwd<HD, ATTN_MAX_KEYS / 16, 4>), dim3((uint32_t)((a.tq + 63) / 64), a.bh), dim3(256), 0, s, a);
}

template <int HD>
void backward_hd(hipStream_t s, const AttnArgs& a) {
  if (waves_for(a, a.tq) == 8)
    hipLaunchKernelGGL((k_attn_bwd_q<HD, 8>), dim3((uint32_t)((a.tq + 127) / 128), a.bh), dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL((k_attn_bwd_q<HD, 4>), dim3((uint32_t)((a.tq + 63) / 64), a.bh), dim3(256), 0, s, a);
  if (waves_for(a, a.tk) == 8)
    hipLaunchKernelGGL((k_attn_bwd_kv<HD, 8>), dim3((uint32_t)((a.tk + 127) / 128), a.bh), dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL((k_attn_bwd_kv<HD, 4>), dim3((uint32_t)((a.tk + 63) / 64), a.bh), dim3(256), 0, s, a);
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

void attention_forward(hipStream_t s, const AttnArgs& a) {
  if (a.mask) {
    const uint64_t n = attention_mask_words(a);
    hipLaunchKernelGGL(k_attn_mask_bits, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, a, a.mask_strides[1] ? a.heads : 1u, n);
  }
  if (a.hd == 16) forward_hd<16>(s, a);
  else if (a.hd == 32) forward_hd<32>(s, a);
  else forward_hd<64>(s, a);
}

void attention_backward(hipStream_t s, const AttnArgs& a) {
  if (a.hd == 16) backward_hd<16>(s, a);
  else if (a.hd == 32) backward_hd<32>(s, a);
  else backward_hd<64>(s, a);
}

}  // namespace rgk
