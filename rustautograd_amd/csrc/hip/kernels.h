// Host-side launchers of the precompiled CDNA4 kernels (kernels.hip, gemm.hip).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "../../../include/rg_plan.h"

namespace rgk {

constexpr int MAX_DIMS = 8;

// Division by a runtime constant through a multiply-high and a shift (Granlund & Montgomery,
// "Division by invariant integers using multiplication", PLDI 1994), valid for n < 2^31.
struct FastDiv {
  uint32_t d = 1, mul = 0, shift = 0;
  FastDiv() = default;
  explicit FastDiv(uint32_t div) : d(div) {
    uint32_t l = 0;
    while ((1ull << l) < div) l++;
    uint64_t p = 31 + l;
    mul = (uint32_t)(((1ull << p) + div - 1) / div);
    shift = (uint32_t)(p - 32);
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const { return d == 1 ? n : (__umulhi(n, mul) >> shift); }
};

// An output index space of up to MAX_DIMS dims and, per operand, the flat stride of each dim.
struct Strided {
  int rank = 0;
  FastDiv size[MAX_DIMS];   // dim sizes, innermost last
  uint32_t st[3][MAX_DIMS];  // strides of up to three operands
  uint32_t base[3] = {0, 0, 0};
};

// Builds `Strided` for an output shape and up to three operand stride lists, merging adjacent
// dims that are contiguous for every operand and dropping size-1 dims.
Strided make_strided(const std::vector<int64_t>& shape, const std::vector<std::vector<int64_t>>& strides);
std::vector<int64_t> row_strides(const std::vector<int64_t>& shape);
// Per-dimension element strides of an operand aligned to the output's trailing dims; broadcast dims read stride 0.
std::vector<int64_t> bcast_strides(const std::vector<int64_t>& shape, size_t rank);

void unary(hipStream_t s, int dtype, int op, const void* a, void* d, uint64_t n);
void binary(hipStream_t s, int dtype, int op, const void* a, const void* b, void* d, uint64_t n, int mode, const Strided* g);
void where(hipStream_t s, int esize, const void* c, const void* a, const void* b, void* d, uint64_t n, int dtype);
void gather(hipStream_t s, int esize, const void* src, void* dst, uint64_t n, const Strided& g);
void pad(hipStream_t s, int esize, const void* src, void* dst, uint64_t n, const std::vector<int64_t>& out_shape,
         const std::vector<int64_t>& starts, const std::vector<int64_t>& in_shape);
void concat_piece(hipStream_t s, int esize, const void* src, void* dst, uint64_t outer, uint64_t len, uint64_t total, uint64_t at);
void take(hipStream_t s, int esize, const void* src, const int32_t* idx, void* dst, uint64_t n, uint64_t block,
          uint64_t n_idx, uint64_t dim);
void take_along(hipStream_t s, int esize, const void* src, const int32_t* idx, void* dst, uint64_t n, uint64_t k, uint64_t v);
void take_grad(hipStream_t s, int dtype, const void* ct, const int32_t* idx, void* dst, uint64_t n, uint64_t block,
               uint64_t n_idx, uint64_t dim);
void take_along_grad(hipStream_t s, int dtype, const void* ct, const int32_t* idx, void* dst, uint64_t n, uint64_t k,
                     uint64_t v);
void rand_uniform(hipStream_t s, int dtype, const int32_t* key, void* dst, uint64_t n);
void rand_normal(hipStream_t s, int dtype, const int32_t* key, void* dst, uint64_t n);
void key_split(hipStream_t s, const int32_t* key, int32_t* dst, uint64_t pairs);
void cast(hipStream_t s, int from, int to, const void* a, void* d, uint64_t n);
void argmax(hipStream_t s, int dtype, const void* a, int32_t* d, uint64_t rows, uint64_t v);
void arg_top_k(hipStream_t s, int dtype, const void* a, int32_t* d, uint64_t rows, uint64_t v, uint64_t k);
void cumsum(hipStream_t s, int dtype, const void* a, void* d, uint64_t rows, uint64_t v, bool reverse);

// Reductions over a canonical pattern; see runtime.cpp for how shapes map onto them.
void reduce_rows(hipStream_t s, int dtype, int kind, const void* a, void* d, uint64_t rows, uint64_t len);
// With chunks > 1, `partial` holds batch*chunks*k elements; with d == nullptr only the chunk
// partials are written, to be folded by fold_rows or fold_jobs.
void reduce_cols(hipStream_t s, int dtype, int kind, const void* a, void* d, uint64_t batch, uint64_t r, uint64_t k,
                 void* partial, uint64_t chunks);
uint64_t reduce_cols_chunks(int dtype, uint64_t batch, uint64_t r, uint64_t k);
// d[c] = the fold over rows 0 .. rows - 1 of partial[row][c], c < k, rows in order.
void fold_rows(hipStream_t s, int dtype, int kind, const void* partial, void* d, uint64_t rows, uint64_t k);
// Up to FOLD_JOBS f32 folds of that form in one launch of `tiles` blocks (job j covers blocks
// [first_tile, next job's first_tile), one per 64 columns).
constexpr int FOLD_JOBS = 48;
struct FoldJob {
  const float* part;
  float* out;
  uint32_t rows, k, kind, first_tile;
};
struct FoldJobs {
  FoldJob job[FOLD_JOBS];
  uint32_t n;
};
void fold_jobs(hipStream_t s, const FoldJobs& jobs, uint32_t tiles);
// Up to FOLD_JOBS f32 sums over a few long rows in one launch: out[i] = part[0][i] + part[1][i]
// + ... + part[rows - 1][i], rows in order, i < n (a multiple of 4; 16-byte aligned part and out),
// 1024 elements per block (job j covers blocks [first_block, next job's first_block)). The form
// of K-split partial products.
struct WideFold {
  const float* part;
  float* out;
  uint64_t n;
  uint32_t rows, first_block;
};
struct WideFolds {
  WideFold job[FOLD_JOBS];
  uint32_t n;
};
void fold_wide(hipStream_t s, const WideFolds& jobs, uint32_t blocks);
void reduce_general(hipStream_t s, int dtype, int kind, const void* a, void* d, uint64_t out_n, const Strided& outer,
                    const Strided& inner, uint64_t red_n);

// Run-loop helpers.
void copy_bytes(hipStream_t s, void* dst, const void* src, uint64_t bytes);
void record_history(hipStream_t s, int dtype, const void* slot, double* hist, const uint64_t* counter, uint64_t stride);
void load_batch(hipStream_t s, void* dst, const void* batches, uint64_t bytes, uint64_t n_batches, const uint64_t* counter);
void counter_inc(hipStream_t s, uint64_t* counter);
// Sets the step counter with a one-thread kernel (no memset node where a caller may capture).
void set_counter(hipStream_t s, uint64_t* counter, uint64_t value);
// Keeps stream `s` busy for about `microseconds` (a bounded wait on the device wall clock).
void hold_stream(hipStream_t s, double microseconds);
void fill_zero(hipStream_t s, void* dst, uint64_t bytes);
// Several copies in one launch: job j copies words[j] 32-bit words from src[j] to dst[j]. No
// job's destination may overlap another job's source or destination.
constexpr int COPY_JOBS = 16;
struct CopyJobs {
  uint32_t* dst[COPY_JOBS];
  const uint32_t* src[COPY_JOBS];
  uint64_t words[COPY_JOBS];
  int n;
};
void copy_batch(hipStream_t s, const CopyJobs& jobs);
// dst[0] = value, with a one-thread kernel.
void set_i32(hipStream_t s, int32_t* dst, int32_t value);

// Dense products. A is [M,K] (or [K,M] when ta), B is [K,N] (or [N,K] when tb), C is [M,N],
// all row-major, over `batch` matrices at the given element offsets (nullptr = contiguous).
struct GemmArgs {
  int dtype;
  bool ta, tb;
  uint64_t m, n, k, batch;
  const void* a;
  const void* b;
  void* c;
  const int64_t* a_off;  // device arrays of per-batch element offsets, or nullptr
  const int64_t* b_off;
  bool a_off4, b_off4;          // every offset in the array is a multiple of 4 elements
  uint64_t a_stride, b_stride;  // per-batch element strides when the offset arrays are null
  void* workspace;              // split-K partial sums, [batch][splits][M N]
  uint64_t workspace_bytes;
  bool defer_split = false;  // leave the partials for fold_wide instead of summing them into C
  int planned_splits = 0;    // with defer_split: the split count the fold was sized for
  const void* bias = nullptr;  // f32 only: bias[c] added to column c of the finished product
};
// Fused attention (attention.hip) over bh = batch * heads independent (tq x hd, tk x hd)
// problems. Operands are strided views: row t of problem b * heads + h starts at
// p + b * sb + h * sh + t * st, with hd contiguous floats (16-byte aligned). The mask, when
// present, is read at b * s0 + h * s1 + q * s2 + k * s3 (zero strides for broadcast dimensions);
// the forward packs it into `mask_bits` (attention_mask_words words), which the backward and
// later forwards over the same mask read.
constexpr int ATTN_MAX_KEYS = 256;
struct AttnOperand {
  const float* p;
  int64_t sb, sh, st;
};
struct AttnArgs {
  uint32_t bh, heads;
  int tq, tk, hd;
  AttnOperand q, k, v;
  const float* mask;
  int64_t mask_strides[4];
  uint32_t* mask_bits;
  float div, fill;  // scores are divided by `div`; masked scores are `fill`
  AttnOperand o;    // forward output
  // Per-query statistics, [bh][tq] each: the row max and sum (forward) and rowsum(dO * O)
  // (backward's query pass).
  float *stat_m, *stat_z, *stat_dd;
  AttnOperand o_in, d_o;  // backward inputs: the forward output and its cotangent
  AttnOperand dq, dk, dv;
  // Optional, backward: column sums of dq, dk and dv over each batch element's rows, as partial
  // rows colp[b][col_len] (a bias gradient of the projection the three share: dq's column c of
  // head h at col_q + h * dq.sh + c, dk's and dv's likewise), for a fold to sum over b. Only with
  // attention_backward_column_sums.
  float* colp = nullptr;
  int64_t col_len = 0, col_q = 0, col_k = 0, col_v = 0;
};
bool attention_supported(int dtype, int64_t hd, int64_t tq, int64_t tk);
uint64_t attention_mask_words(const AttnArgs& a);
// `build_mask_bits`: pack the mask into `mask_bits` first (else they hold it already).
void attention_forward(hipStream_t s, const AttnArgs& a, bool build_mask_bits = true);
void attention_backward(hipStream_t s, const AttnArgs& a);
// Whether the backward of these shapes can write column sums (AttnArgs::colp): one block per
// problem for each pass, which holds all of the problem's rows.
bool attention_backward_column_sums(const AttnArgs& a);

// Whether the product runs through the bandwidth-bound skinny kernels (alignment aside: an
// unaligned operand falls back to the general kernels at launch).
bool gemm_streamed(int dtype, uint64_t m, uint64_t n, uint64_t k, uint64_t batch, bool ta, bool tb);

// The number of K splits the product runs with (1: none), and the workspace bytes its split-K
// partials need.
int gemm_splits(int dtype, uint64_t m, uint64_t n, uint64_t k, uint64_t batch, bool ta, bool tb);
uint64_t gemm_workspace(int dtype, uint64_t m, uint64_t n, uint64_t k, uint64_t batch, bool ta, bool tb);

// The MFMA tile of a single (unbatched) fp32 product whose operands are 16-byte aligned, as plan
// slots are, when it runs unsplit on the tile kernel and each lane's finished outputs come in
// runs of two or four adjacent columns (the form an elementwise epilogue takes): the shape
// arguments of the tile kernel (gemm_mfma.h). False for any other product. `mode` is the tile's
// load mode, GEMM_WHOLE_TILES when M, N and K are multiples of the tile.
constexpr int GEMM_WHOLE_TILES = 0;  // rgg::LOAD_EVEN
struct GemmTile {
  int bm, bn, bk, wm, wn, ms, mode, kps;
  uint32_t tm, tn;
};
bool gemm_epilogue_tile(int dtype, uint64_t m, uint64_t n, uint64_t k, bool ta, bool tb, GemmTile* t);
void gemm(hipStream_t s, const GemmArgs& g);
// Two or three independent products in one launch, when all are unbatched MFMA tile products
// on the same tile shape (with a sequence of operand layouts instantiated for it), every
// operand's vectors inside its tile grid and any K split deferred to the fold area; false,
// launching nothing, otherwise. With `launch` false it only answers (operand pointers may be
// null).
bool gemm_group(hipStream_t s, const GemmArgs* g, int count, bool launch = true);

}  // namespace rgk
