// Fused elementwise groups as JIT-compiled kernels: one kernel per group, specialised to its
// micro-op chain, input kinds, shape and element count (all compile-time constants), compiled
// for gfx950 with hiprtc. The reference compiles one MSL function per group body for the same
// reason (src/metal.rs:122-152, 455-479).
#pragma once
#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "../../../include/rg_plan.h"

namespace rgjit {

constexpr int TPB = 256;

struct FusedKernel {
  std::string name;
  uint32_t grid = 0;     // blocks of TPB threads
  int vec = 1;           // elements per thread
  hipFunction_t fn = nullptr;
  // Row groups with column reductions: per output, the reduce kind of a column output (-1 for
  // the others), which the kernel writes as `grid` partial rows of row_len values to be folded.
  std::vector<int> col_kind;
  uint32_t row_len = 0;
  uint32_t block = TPB;  // threads per block
};

// A row group with column reductions: COL_BLOCKS blocks of COL_WAVES waves (one block per CU,
// four waves per SIMD), each folding the rows it walks into one partial row. (Two blocks per CU
// at 64 registers, one row per wave, measured no faster on C4's layer norms.)
constexpr int64_t COL_BLOCKS = 256;
constexpr int COL_WAVES = 16;
// Column reductions of one group staged in LDS together when they take at most this many bytes.
constexpr uint64_t COL_LDS_BYTES = 64 * 1024;

// Source of one kernel named `name` computing group `f` (`k->grid` blocks). Outputs whose slot is
// also an input slot are written in place (each element is read before it is written). With
// `device_fn`, the source is instead a device function `name(block, inputs..., outputs...)` that
// computes the elements of block `block`.
std::string generate(const rgplan::Fused& f, const std::string& name, FusedKernel* k, bool device_fn = false);

// Source of one kernel computing several independent groups side by side (horizontal fusion):
// blocks [start_j, start_j + grid_j) compute part j. For groups too small to fill the device on
// their own.
// Its parameters are the distinct slots of the parts (merged_slots: inputs then outputs, part after
// part, each slot once), so operands the parts share, such as an optimizer's scalars, pass once.
std::string generate_merged(const std::vector<const rgplan::Fused*>& parts, const std::string& name, FusedKernel* k);
std::vector<int64_t> merged_slots(const std::vector<const rgplan::Fused*>& parts);

// Source of one row-group kernel (RG_STEP_ROWS): `k->grid` blocks of four rows each, or, with
// column reductions, COL_BLOCKS blocks of COL_WAVES waves walking the rows grid-stride and writing
// one partial row per block for each column output (see col_kind).
std::string generate_rows(const rgplan::Fused& f, const std::string& name, FusedKernel* k);

// A product's tile for generate_gemm (the template arguments of rgg::gemm_mfma_block).
struct ProductTile {
  int bm, bn, bk, wm, wn, ms, mode;
  bool ta, tb;
};

// Source of one product kernel whose epilogue computes fused group `f` (a plain fused group over
// the product's M x N outputs, reading the product through `c_slot`) from each finished output
// before it is stored: the tile of gemm_mfma.h with an epilogue that loads the group's other
// inputs at the output's position, applies its operations in its order (the values the plain
// group kernel would compute) and stores its outputs, and the product itself when `store_c`.
// The kernel's parameters are the tile kernel's, then the epilogue's pointers (product, the
// group's inputs in order, its outputs in order). With `col_sum` >= 0 the kernel also sums
// output `col_sum` over its tile's rows, column by column, once its outputs are stored, and
// writes one partial row per tile row to a last pointer parameter: partial [tile row][N],
// summed in tile-row order by a fold (a column sum that reads the group's output, computed here
// instead of re-reading it).
std::string generate_gemm(const rgplan::Fused& f, int64_t c_slot, bool store_c, const ProductTile& t, const std::string& name,
                          FusedKernel* k, int col_sum = -1);

// Compiles all sources into one code object for gfx950 and resolves each kernel. Modules are
// cached by source text for the life of the process. Throws std::runtime_error with the log.
void compile(const std::string& source, std::vector<FusedKernel*>& kernels);

// The gfx950 code object for `source` (ops prelude added); throws with the compiler log.
std::vector<char> compile_code(const std::string& source);

}  // namespace rgjit
