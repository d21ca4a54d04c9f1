/* rg HIP device backend: the C ABI of librg_hip.so.
 *
 * This is the drop-in replacement for rg's device layer. In the reference that layer is the
 * `Exec` trait (src/plan.rs:29-41) implemented by `MetalExec` (src/metal.rs:728-750), built by
 * `MetalProgram` (src/metal.rs:362-530), stubbed on other platforms by src/metal_stub.rs:6-40
 * and selected in src/lib.rs:4-8. Each entry point below names the reference interface it
 * replaces. Plans arrive as the flat descriptor of rg_plan.h.
 *
 * Ownership: a program owns the device kernels, the step list and a pool of slot frames; an
 * exec owns one frame and returns it to the pool when freed (metal.rs:505-523, 565-571).
 * Errors: construction reports a message through (err, err_len); execution errors are latched,
 * the first one wins and later steps do nothing until the exec is freed (metal.rs:536-537,
 * 584-590). Threading: a program may be shared; each exec is used by one thread at a time.
 */
#ifndef RG_HIP_H
#define RG_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "rg_plan.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The device-resident step loop: the arguments of `run_loop` (src/validate.rs:289-363) after
 * the engine has derived its swap and copy lists from the plan (validate.rs:303-318). */
typedef struct rg_run_desc {
  int64_t n_swaps;
  const int64_t* swaps;        /* n_swaps pairs (input slot, output slot): buffers exchanged */
  int64_t n_copies;
  const int64_t* copies;       /* n_copies triples (input slot, output slot, elements) */
  int64_t n_data;
  const int64_t* data_slots;   /* slots of the data inputs */
  const uint64_t* data_bytes;  /* bytes of each data input */
  int64_t n_batches;           /* >1: batch k % n_batches is loaded before step k */
  const void* const* batches;  /* host pointers, batches[b * n_data + j] */
  int64_t n_history;
  const int64_t* history_slots;/* scalar outputs recorded after every step */
  int64_t steps;
  double* history;             /* out: n_history rows of `steps` values */
} rg_run_desc;

typedef struct rg_run_result {
  int64_t done;                /* completed steps */
  int64_t nonfinite_step;      /* first step whose history held a non-finite value, or -1 */
  double seconds;              /* wall seconds of the loop itself; setup and transfers not counted */
} rg_run_result;

/* metal.rs:58-60 `available()`: 1 when a gfx950 device is present. */
int rg_hip_available(void);
/* Total HBM of device 0 in bytes, for the planner's memory warning (no reference counterpart;
 * the reference asks the OS for physical memory, python/rg/_core.py:939-955). */
uint64_t rg_hip_device_memory_bytes(void);
/* Generates and compiles the JIT kernels of every fused group of a plan for gfx950 without a
 * device; returns the kernel count or -1 with the compiler log. No reference counterpart: it
 * checks the code generator in build environments without a GPU. */
int rg_hip_compile_check(const int64_t* plan_words, size_t n_words, char* err, size_t err_len);

/* metal.rs:380-503 `MetalProgram::new(&Plan)`: builds the kernels for every plan step (JIT
 * compiled fused groups plus precompiled instruction kernels). Refuses a slot larger than the
 * device memory. Returns NULL with a message on failure (validate.rs:478-482 turns it into
 * DEVICE_UNAVAILABLE). */
void* rg_hip_program_new(const int64_t* plan_words, size_t n_words, const void* const_blob,
                         size_t const_bytes, char* err, size_t err_len);
void rg_hip_program_free(void* program);
/* metal.rs:385-388 `allocated_bytes()`: device bytes this process holds, to catch leaks. */
uint64_t rg_hip_program_allocated_bytes(void* program);
/* No counterpart in the reference (its Metal backend runs every plan step as its own dispatch):
 * the plan step whose kernel computes `step`. A product that runs a following elementwise group
 * in its epilogue computes both; the one of the two that does not launch anything returns the
 * other, every other step itself; -1 for a step out of range. For per-step timing and rooflines. */
int64_t rg_hip_program_step_runs_in(void* program, int64_t step);
/* metal.rs:525-529 `inject_failure_for_test()`: the next step fails as a device error would. */
void rg_hip_program_inject_failure(void* program);
/* Test hook next to `inject_failure_for_test` (metal.rs:525-529), with no reference counterpart:
 * the next `steps` plan passes complete and the one after fails, as a device error would, so a
 * test can check what a failure in the middle of a run hands back. The failure is latched on the
 * host side; no device fault is involved. */
void rg_hip_program_inject_failure_after(void* program, int64_t steps);

/* metal.rs:505-523 `MetalProgram::exec`: a frame from the pool, or a new zeroed one with the
 * constants written. */
void* rg_hip_exec_new(void* program, char* err, size_t err_len);
/* Drop of `MetalExec` (metal.rs:565-571): the frame goes back to the pool. */
void rg_hip_exec_free(void* exec);
/* `Exec::write_prefix` / `Exec::load` (plan.rs:33, 36): host bytes into the start of a slot. */
int rg_hip_exec_write(void* exec, int64_t slot, const void* src, uint64_t bytes);
/* `Exec::prefix` (plan.rs:35): the first bytes of a slot back to the host. */
int rg_hip_exec_read(void* exec, int64_t slot, void* dst, uint64_t bytes);
/* `Exec::load` for many slots at once (run_loop's state load, validate.rs:290-292): every copy is
 * enqueued, then one wait; a batch of at least 1 MiB passes through the frame's pinned staging
 * (filled on several host threads, then one DMA per slot), so `srcs` may be pageable memory.
 * Returns 0, or -1 for a bad slot or size (nothing copied) or a failure. */
int rg_hip_exec_write_slots(void* exec, int64_t n, const int64_t* slots, const void* const* srcs, const uint64_t* bytes);
/* `Exec::prefix` for many slots at once (run_loop's final state read, validate.rs:361): every
 * copy is enqueued, then one wait (through the staging as above, drained after the wait).
 * Returns as rg_hip_exec_write_slots. */
int rg_hip_exec_read_slots(void* exec, int64_t n, const int64_t* slots, void* const* dsts, const uint64_t* bytes);
/* `Exec::scalar` (plan.rs:37): element 0 of a slot as a double. */
double rg_hip_exec_scalar(void* exec, int64_t slot);
/* `Exec::swap` (plan.rs:34): exchanges the buffers behind two slots. */
void rg_hip_exec_swap(void* exec, int64_t a, int64_t b);
/* `Exec::step` (plan.rs:32): runs every plan step once and waits for the device (synchronous:
 * a failure is visible to rg_hip_exec_failure when it returns). */
void rg_hip_exec_step(void* exec);
/* Runs plan steps [begin, end) and waits: what the instrumented check needs between steps. */
void rg_hip_exec_steps(void* exec, int64_t begin, int64_t end);
/* `Exec::failure` (plan.rs:38-40): 1 and the message when the device failed, else 0. */
int rg_hip_exec_failure(void* exec, char* buf, size_t len);
/* metal.rs:690-698 `step_timed`: adds each plan step's device seconds to seconds[step]. */
int rg_hip_exec_step_timed(void* exec, double* seconds);
/* metal.rs:700-713 `breakdown`: whole steps, and where the time went, as JSON. */
int rg_hip_exec_breakdown(void* exec, int64_t repeats, char* json, size_t len);
/* Measurement helper next to `step_timed` (metal.rs:690-698), with no reference counterpart:
 * runs the listed plan steps back to back, `repeats` times, between two HIP events on the
 * execution stream, and stores the elapsed seconds. Gives a kernel class's average launch
 * duration without per-step event overhead. Slot contents afterwards are unspecified. */
int rg_hip_exec_time_steps(void* exec, const int64_t* steps, int64_t n_steps, int64_t repeats, double* seconds);
/* The generated HIP source of every fused kernel of a plan (its control-flow bodies included),
 * for inspection; touches no device. Returns the kernel count, -2 when `len` is too small (the
 * source is cut), or -1 with the message in `buf`. No reference counterpart. */
int rg_hip_kernel_source(const int64_t* words, size_t n_words, char* buf, size_t len);
/* Roofline support for `Compiled::profile` (validate.rs:875-919 times operations; this adds the
 * ceiling they are measured against), with no reference counterpart. Whether the backend runs
 * a product of op(A) m x k by op(B) k x n over `batch` problems through its bandwidth-bound
 * streaming kernels (1) or its matrix-core kernels (0): a pure function of the arguments that
 * touches no device. */
int rg_hip_gemm_streamed(int32_t dtype, int64_t m, int64_t n, int64_t k, int64_t batch, int32_t ta, int32_t tb);
/* The current device's published peaks: peaks[0] HBM bandwidth in GB/s, peaks[1] dense fp32
 * matrix-core TFLOP/s, peaks[2] dense fp64 matrix-core TFLOP/s, and its name in `name`.
 * Returns 0, or 1 (message in `name`) when no device is visible or it has no published figures. */
int rg_hip_device_peaks(double* peaks, char* name, size_t len);
/* The device-resident `run_loop` (validate.rs:289-363): steps captured in HIP graphs and
 * replayed, batches and history kept on the device, state handed off by buffer swaps and
 * copies. Semantics equal the host loop: a non-finite history value stops the run after that
 * step's state handoff. Returns 0, or -1 when the device failed (see rg_hip_exec_failure); the
 * state slots then hold the state after `out->done` steps, as in the host loop. The captured
 * graphs and the loop's device buffers stay with the frame and are reused by the next run with
 * the same description. `out->seconds` is the step loop alone (validate.rs:264-265): batch
 * upload and graph capture are excluded. A description whose slot indices, counts, sizes or
 * pointers do not fit the program (swaps of unequal or shared slots, copies or data larger than
 * their slots, a missing batch pointer or history buffer) is refused with -1 and a message
 * before anything is copied or launched. */
int rg_hip_exec_run(void* exec, const rg_run_desc* desc, rg_run_result* out);
/* The step loop of rg_hip_exec_run for callers that cannot allocate device memory (code that
 * must not call hipMalloc: tight serving loops, harnesses that forbid it). It has no counterpart
 * in the reference. It calls no hipMalloc, hipFree or other allocating routine and instantiates
 * no graph: the run's step counter, history record, cycled batches and state-copy temporaries
 * live in a static device array of RG_NOALLOC_SCRATCH_BYTES (32 MiB) that each GPU holds until
 * the process ends, and the steps are launched directly. A run whose buffers would exceed it is
 * refused (-1, message in rg_hip_exec_failure) before anything runs. Results equal
 * rg_hip_exec_run's, bit for bit, and descriptions are checked as there. With history it waits
 * after every step to check the recorded values. `out->done` counts the steps a successful
 * synchronization confirmed: without history that is the final one, so a device failure it
 * reports gives 0. Every call on one GPU shares that GPU's array and leaves its contents behind;
 * a per-device lock held for the whole call makes calls that overlap on one GPU take turns. It
 * keeps no snapshot: after a device failure the state slots are unspecified. */
int rg_hip_exec_run_noalloc(void* exec, const rg_run_desc* desc, rg_run_result* out);

#ifdef __cplusplus
}
#endif

#endif /* RG_HIP_H */
