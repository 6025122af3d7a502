/*
 * libtempest_hip — the C ABI of Tempest's MI355X (gfx950) execution backend.
 *
 * One process drives one GPU.  Every entry point returns an int status:
 * TH_OK (0) on success, otherwise a TH_E_* code or a positive hipError_t;
 * th_last_error() then holds a message for the calling thread.  Pointers are
 * device addresses unless the name says host.  Arrays are the reference's
 * dense column-major layout (first axis fastest, src/Compiler/IR/layout.jl:1-3);
 * "rows" below are therefore the reference's columns: a reduction over
 * `dims = 1` of an n x rows array is a reduction over contiguous runs of n.
 *
 * Each declaration names the reference interface it replaces (paths are
 * relative to the Tempest.jl source tree).  A Julia extension binds these by
 * `ccall`; the host mirror in tempest.jl_amd/tempest_hip binds them by ctypes.
 */
#ifndef TEMPEST_HIP_H
#define TEMPEST_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  TH_OK = 0,
  TH_E_ARGUMENT = -1,     /* shapes, strides or alignment a kernel cannot take */
  TH_E_STATE = -2,        /* no th_init, or a handle used after release        */
  TH_E_UNSUPPORTED = -3,  /* a case this build does not implement              */
  TH_E_MEMORY = -4,       /* an allocation failed                              */
  TH_E_COMPILE = -5       /* a generated kernel failed to compile              */
};

typedef struct th_launch th_launch; /* one claim's built launch: kernels + arguments */
typedef struct th_graph th_graph;   /* a captured run of launches                   */
typedef struct th_arena th_arena;   /* the slot arena: one device slab              */

/* Device rates as the cover prices them.
 * Replaces device_rates(::CUDATarget), ext/CUDAExt.jl:913-921. */
typedef struct th_rates {
  double launch;    /* seconds between launches inside a replayed graph:
                       an empty kernel's share of a long one (measured)    */
  double cached;    /* bytes/s read from what L2 + MALL hold (measured)      */
  double bandwidth; /* bytes/s from HBM (memory clock x bus width)           */
  double cache;     /* bytes of last-level cache (L2 + MALL)                 */
  double blocks;    /* workgroups that fill the device (CUs)                 */
} th_rates;

/* Algorithmic work of one launch, as Implement.Work states it
 * (src/Compiler/Implement/Implement.jl:61-82): the bytes a launch must move
 * and the flops it must do, whatever its tiling. */
typedef struct th_work {
  double bytes;
  double flops;
  int64_t blocks;    /* workgroups launched by the dominant kernel */
  int32_t kernels;   /* kernels in the launch                      */
  int32_t values;    /* repointable values (see th_launch_repoint) */
} th_work;

/* ---- errors, device, streams ------------------------------------------- */

/* The last failure's message on this thread; "" when none. */
const char* th_last_error(void);

/* Make `device` current and create the library's stream on it.
 * Replaces task_state/on_device(::CUDATarget), ext/CUDAExt.jl:18-22,44-48. */
int th_init(int device);

/* Wait for the device and release the library's stream and helpers. */
int th_shutdown(void);

/* The device's marketing name and gfx arch, e.g. "AMD Instinct MI355X (gfx950)".
 * Replaces device_name(target), src/Compiler/runtime/target.jl:583-584. */
int th_device_name(char* host_out, size_t capacity);

/* "hip=<runtime version>;clang=<compiler>;arch=gfx950".
 * Replaces toolchain(target), src/Compiler/runtime/target.jl:594. */
int th_toolchain(char* host_out, size_t capacity);

/* Replaces device_rates(::CUDATarget), ext/CUDAExt.jl:906-921. */
int th_device_rates(th_rates* host_out);

/* Run the library's launches on `stream`, a hipStream_t (NULL is the null
 * stream).  th_init starts on a non-blocking stream of the library's own,
 * which th_get_stream returns until another is set.
 * Replaces stream/task_stream(::CUDATarget), ext/CUDAExt.jl:326-337. */
int th_set_stream(void* stream);
int th_get_stream(void** host_out);

/* Wait until the stream has run everything launched on it.
 * Replaces quiesce(target[, stream]), src/Compiler/runtime/target.jl:493,617. */
int th_quiesce(void);

/* ---- storage --------------------------------------------------------------- */

/* A device buffer of `bytes`, 256-byte aligned.
 * Replaces allocate(::CUDATarget, T, n), ext/CUDAExt.jl:23. */
int th_alloc(size_t bytes, void** host_out);
int th_free(void* ptr);

/* Host -> device, device -> host and device -> device copies on the stream;
 * th_download waits for its copy.  Replace upload!/download!
 * (src/Compiler/runtime/target.jl:258,267; ext/CUDAExt.jl:31-34) and the
 * runtime's Copy (src/Compiler/runtime/runtime.jl:47-64). */
int th_upload(void* dst, const void* host_src, size_t bytes);
int th_download(void* host_dst, const void* src, size_t bytes);
int th_copy(void* dst, const void* src, size_t bytes);

/* A device-to-device copy of `bytes` bytes as a launch: run it, record it in
 * a graph and repoint it as any other (values: 0 dst, 1 src; any alignment).
 * Replaces the `Copy` step (src/Compiler/runtime/runtime.jl:47-64) where a
 * target records its steps as one graph (capture, ext/CUDAExt.jl:515-572,
 * records a copy node for it). */
int th_build_copy(void* dst, const void* src, uint64_t bytes, th_launch** host_out);

/* The slot arena: `n` slots of `sizes[i]` bytes laid out in one hipMalloc
 * slab, each at a multiple of `align` (>= 256, a power of two).  Replaces the
 * per-slot allocate of `planned`, src/Compiler/runtime/runtime.jl:415, fed by
 * the planner's Storage.sizes (src/Compiler/plan/storage.jl:37-46). */
int th_arena_create(const uint64_t* host_sizes, int n, uint64_t align, th_arena** host_out);
int th_arena_slot(th_arena* arena, int slot, void** host_out);
int th_arena_bytes(th_arena* arena, uint64_t* host_out);
int th_arena_destroy(th_arena* arena);

/* The slot pool: one reserved range of `reserve` bytes of device addresses
 * (hipMemAddressReserve), mapped to memory (hipMemCreate, hipMemMap) as
 * blocks are taken; without virtual memory management, one allocation of
 * that size.  th_pool_alloc takes a block (first fit, else past the highest
 * block, 256-byte or `align`-aligned); th_pool_free returns it.  Every block
 * lies in [base, base + reserved): the planner's slots, allocated one by one
 * as `planned` does (src/Compiler/runtime/runtime.jl:415, allocate(t, T, n)
 * per slot), land in one range.  Replaces allocate(::CUDATarget, T, n),
 * ext/CUDAExt.jl:23, for the slots of an executable.  th_pool_destroy waits
 * for the device and unmaps everything — at once when no block is taken,
 * else when th_pool_free returns the last one (no block may be taken after
 * it), so a host whose collector frees the pool before its buffers (Julia
 * finalizes objects that die together in no set order) frees no memory
 * still in use.  The pool calls are safe from several threads. */
typedef struct th_pool th_pool;
int th_pool_create(uint64_t reserve, th_pool** host_out);
int th_pool_alloc(th_pool* pool, uint64_t bytes, uint64_t align, void** host_out);
int th_pool_free(th_pool* pool, void* ptr);
int th_pool_info(th_pool* pool, void** host_base, uint64_t* host_reserved, uint64_t* host_mapped);
int th_pool_destroy(th_pool* pool);

/* ---- launches ---------------------------------------------------------- */

/* Run a launch's kernels on the stream, in order: a step of `execute!`.
 * Replaces (l::FloorLaunch)(), ext/CUDAExt.jl:1092-1098, and the claims'
 * launch calls (src/Compiler/runtime/schedule.jl:131-136). */
int th_launch_run(th_launch* launch);

/* Point value `value` of a launch at `ptr`, as its builder numbered the
 * values.  Replaces Implement.repoint!(launch, value, buffer),
 * src/Compiler/Implement/Implement.jl (repoint!), ext/CUDAExt.jl:1086-1090. */
int th_launch_repoint(th_launch* launch, int value, void* ptr);

/* The launch's algorithmic work.  Feeds Implement.estimate,
 * src/Compiler/Implement/Implement.jl:61-82. */
int th_launch_work(th_launch* launch, th_work* host_out);

/* A one-line description (kernel names and grids), as build_claim's
 * description string (src/Compiler/Implement/Implement.jl, build_claim). */
int th_launch_describe(th_launch* launch, char* host_out, size_t capacity);

int th_launch_destroy(th_launch* launch);

/* A launch's workspace: the bytes of device memory its kernels use beyond its
 * values (partial sums, statistics, stored intermediates such as attention's
 * dS'), 0 for none.  Builders allocate nothing: a launch without a workspace
 * given allocates it at its first run or capture and owns it;
 * th_launch_set_workspace gives it memory of the caller's instead (256-byte
 * aligned, at least th_launch_workspace bytes, alive while the launch runs),
 * freeing one it owned.  A graph captured before must be retargeted
 * (th_graph_retarget).  This lets a planner place workspaces in its arena
 * beside the slots (`planned`'s allocations, src/Compiler/runtime/runtime.jl:415),
 * as the reference's floor takes its workspaces from the target
 * (allocate(target, ...) in build_floor, src/Compiler/runtime/runtime.jl:1326-1327). */
int th_launch_workspace(th_launch* launch, uint64_t* host_bytes);
int th_launch_set_workspace(th_launch* launch, void* ptr);

/* ---- graphs ------------------------------------------------------------ */

/* Record `n` launches, in order, as one graph of kernel nodes.
 * Replaces capture(::CUDATarget, steps, keep), ext/CUDAExt.jl:515-572. */
int th_graph_capture(th_launch* const* host_steps, int n, th_graph** host_out);

/* Launch the graph on the stream.  Replaces replay(::CUDATarget, graph),
 * ext/CUDAExt.jl:739. */
int th_graph_replay(th_graph* graph);

/* Make the graph read what step `step`'s launch now reads, after
 * th_launch_repoint moved its values: the step's kernel nodes take the
 * launch's current arguments in place.  Replaces retarget!(::CUDATarget,
 * graph, steps, moves, repoint) and patch!, ext/CUDAExt.jl:604-668. */
int th_graph_retarget(th_graph* graph, int step);

/* Replaces release(::CUDATarget, graph), ext/CUDAExt.jl:743. */
int th_graph_release(th_graph* graph);

/* ---- measuring --------------------------------------------------------- */

/* Device seconds of one run of `launch` replayed alone as a graph after the
 * caches are cleared (a read of 2 x (L2 + MALL)), the minimum over `samples`
 * (0 = chosen as the reference does), less what replaying one graph adds.
 * Replaces time_launch/timed_launch/cleared/replay_overhead,
 * ext/CUDAExt.jl:760-882. */
int th_time_launch(th_launch* launch, int samples, double* host_seconds);

/* Mean device seconds of one replay of `graph`, `reps` replays back to back
 * between two events (warm caches), after `warmup` replays.  Replaces
 * batched(target, launch), ext/CUDAExt.jl:886-898. */
int th_time_graph(th_graph* graph, int warmup, int reps, double* host_seconds);

/* Mean device seconds of one run of `launch` (warm), as th_time_graph. */
int th_time_run(th_launch* launch, int warmup, int reps, double* host_seconds);

/* What dispatch costs on this device, measured once per process with an
 * empty kernel, each the mean of a long back-to-back run: `graph_base`, what
 * replaying a graph costs beyond its launches; `in_graph`, one launch inside a
 * replayed graph (th_rates.launch); `direct`, one launch made directly.  A
 * recording of K launches replays faster as a graph when
 * graph_base + K in_graph < K direct, else as its launches one by one.
 * Extends replay_overhead and LAUNCH, ext/CUDAExt.jl:874-906, whose target
 * always records a graph (capture(::CUDATarget, ...), ext/CUDAExt.jl:565). */
int th_dispatch_costs(double* graph_base, double* in_graph, double* direct);

/* The matrix cores' sustained bf16 rate on this device, measured: every SIMD
 * runs two waves of back-to-back v_mfma_f32_32x32x16_bf16 on register
 * operands, one operand pair throughout (vary = 0) or eight pairs of random
 * bits cycled so that each product's operands differ (vary = 1, as real
 * data's do); flop/s over the run, and the shader clock the waves ran at
 * (their clock counter against the 100 MHz real-time counter).  The ceiling
 * any product kernel meets on this device, beside the data-sheet peak.  No
 * reference counterpart: the reference fits product rates from products
 * (cover/calibrate.jl). */
int th_matrix_rate(int vary, double* host_flops_per_s, double* host_clock_hz);

/* The LDS read rate on this device, measured: workgroups of four waves (one
 * or two a CU, per_cu) read 64 KB of LDS in a loop, eight 1 KB wave reads in
 * flight, by ds_read_b128 (mode 0) or pairs of ds_read_b64_tr_b16 (mode 1);
 * modes 2 and 3 issue one v_mfma_f32_32x32x16_bf16 on each read as well (32
 * flops a byte, the attention sweeps' ratio).  Bytes/s and flop/s over the
 * run, and the shader clock the waves ran at.  The LDS ceiling the attention
 * kernels meet.  No reference counterpart: a device measurement. */
int th_lds_rate(int mode, int per_cu, double* host_bytes_per_s, double* host_flops_per_s, double* host_clock_hz);

/* The HBM read rate on this device, measured: one workgroup of four waves a
 * CU, each wave keeping eight 1 KB loads (non-temporal) in flight, over a
 * 2 MB stream of its own (mode 0) or over the attention dQ sweep's dS' reads
 * at B 8, H 16, S 4096 (mode 1: causal streams of 8 KB steps, two query
 * blocks a workgroup).  Bytes/s over five launches.  The ceiling of the dQ
 * sweep's stream.  No reference counterpart: a device measurement. */
int th_read_rate(int mode, double* host_bytes_per_s);

/* ---- op class (a): fused pointwise + reductions -------------------------- */

/* Softmax over each contiguous run of n (a column of the reference's n x rows
 * array) and its gradient, one program:
 *   y = exp.(x .- logsumexp(x; dims = 1)),  loss = sum(y .* g),
 *   dx = y .* (g .- sum(y .* g; dims = 1)).
 * Inputs x, g (rows x ld floats, ld >= n); outputs dx (same layout) and
 * loss (one float).  The fold is the reference's online softmax
 * (Relative{Exponential}, src/Compiler/IR/folds.jl:119-222) run resident in
 * registers, as the cuTile resident sketch (ext/cuTileExt/build.jl:138,
 * ext/cuTileExt/cuTileExt.jl:638-672).  Values: 0 x, 1 g, 2 dx, 3 loss.
 * The program is test/fixtures/programs.jl:8,74 differentiated. */
int th_build_softmax_grad(int64_t rows, int32_t n, int64_t ld,
                          const float* x, const float* g, float* dx, float* loss,
                          th_launch** host_out);

/* th_build_softmax_grad's program run at once on the library's stream, with
 * no device allocation: no counterpart in the reference.  It is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The per-row loss partials
 * go to a static device scratch of 2^20 floats that each GPU holds until the
 * process ends, so rows must be at most 1048576 (TH_E_ARGUMENT beyond).  Every
 * call on a GPU shares that GPU's scratch: calls that overlap on one GPU (on
 * different streams, or from different threads) race.  The same kernels as
 * th_build_softmax_grad, so the results are bit-identical to its launch's. */
int th_softmax_grad_noalloc(int64_t rows, int32_t n, int64_t ld,
                            const float* x, const float* g, float* dx, float* loss);

/* LayerNorm (weight 1, bias 0) over each contiguous run of n and its
 * gradient: y = (x .- m) ./ sqrt.(v .+ eps) with m, v the run's mean and
 * mean square deviation (two passes, test/fixtures/programs.jl:13-17),
 * loss = sum(y .* g), dx = r .* (g .- mean(g) .- y .* mean(g .* y)),
 * r = 1/sqrt(v + eps).  Values: 0 x, 1 g, 2 dx, 3 loss. */
int th_build_layernorm_grad(int64_t rows, int32_t n, int64_t ld, float eps,
                            const float* x, const float* g, float* dx, float* loss,
                            th_launch** host_out);

/* Forward only: y = softmax(x; dims = 1) (values 0 x, 1 y) and
 * y = layernorm(x) (values 0 x, 1 y), over rows runs of n at stride ld. */
int th_build_softmax_fwd(int64_t rows, int32_t n, int64_t ld, const float* x, float* y,
                         th_launch** host_out);
int th_build_layernorm_fwd(int64_t rows, int32_t n, int64_t ld, float eps, const float* x,
                           float* y, th_launch** host_out);

/* The sum of `count` floats into one (a full reduction, the cuTile `:full`
 * sketch, ext/cuTileExt/cuTileExt.jl:638-641): values 0 x, 1 out. */
int th_build_sum(int64_t count, const float* x, float* out, th_launch** host_out);

/* ---- op class (a), generated: the floor for any pointwise or reduction group
 *
 * A group is a domain of up to four axes (axis 0 fastest), its values (dense
 * one-dimensional buffers), its terms and, for a reduction group, its folds
 * over the axes marked in `reduced`, run in phases.  The library writes a
 * gfx950 kernel for the group (one per phase when the folds' positions split
 * among workgroups), compiles it at run time and keeps the code object in a
 * content-keyed cache on disk ($TEMPEST_HIP_CACHE, else $XDG_CACHE_HOME/
 * tempest_hip, else ~/.cache/tempest_hip).  Replaces the floor's generated
 * kernels: scalar_kernel (codegen/scalar.jl:186-250), split_kernels
 * (scalar.jl:284-348), floor_launch / floor_split / merge_lanes
 * (ext/CUDAExt.jl:926-1017) and the kernel cache (runtime/cache.jl). */

#define TH_FLOOR_RANK 4

/* A scan group sweeps its scanned axes (`reduced`) one item at a time, in
 * order (reversed with TH_FLOOR_REVERSE): at each position every fold takes
 * its element in (phase, index) order, a scan's result there is what later
 * folds and the full outputs read, and the plain folds' results are read by
 * the once outputs after the sweep (scan_kernel, codegen/scalar.jl:350-398). */
enum { TH_GROUP_POINTWISE = 0, TH_GROUP_REDUCTION = 1, TH_GROUP_SCAN = 2, TH_GROUP_RECURRENCE = 3 };
#define TH_FLOOR_REVERSE 1
/* A pointwise group whose items run one after another, in order, on one
 * thread: a fold by key's elements (accumulating outputs) then add without
 * atomics, in the items' order, so every run rounds alike (the CPU floor's
 * order, src/Compiler/codegen/scalar.jl:496-522).  What a deterministic target
 * (src/Compiler/runtime/target.jl:229-231) asks of a fold by key. */
#define TH_FLOOR_ORDERED (1 << 16)

/* A recurrence group (recurrence_kernel, codegen/scalar.jl:402-440) steps
 * along one axis, named by the flags (TH_FLOOR_STEP(axis)), a thread per
 * position of its parallel axes (those not in `reduced`); at each step it
 * computes and stores its outputs in order, each over the positions of the
 * other `reduced` axes its address mentions (the rest at zero), reading what
 * the steps before and this one stored.  An output's `full` field says when
 * it runs: TH_STEP_EACH at every step; TH_STEP_FIRST at the first alone (a
 * state where it starts); TH_STEP_LAST at the last alone; TH_STEP_CARRY at
 * every step but the last, its address already one step on (a value carried
 * into its state for the next step).  A recurrence group has no folds but
 * recomputed ones.  TH_FLOOR_REVERSE steps from the last position. */
#define TH_FLOOR_STEP(axis) ((axis) << 8)
enum { TH_STEP_EACH = 0, TH_STEP_FIRST = 1, TH_STEP_LAST = 2, TH_STEP_CARRY = 3 };

/* Terms (Load, Lit, Ix, Stat, Apply of src/Compiler/IR):
 *   TH_TERM_LOAD   element index(i) of value `ref`, widened to fp32
 *   TH_TERM_LIT    the number `lit`
 *   TH_TERM_INDEX  the fp32 value of the affine expression `index` of the
 *                  domain's zero-based positions
 *   TH_TERM_STAT   fold `ref`'s result, as `observe` reads it
 *   TH_TERM_APPLY  function `fn` of terms args[0..arity) (earlier terms)
 *   TH_TERM_RECOMPUTE  fold `ref` (phase 0) computed where it is read, as
 *                  `observe` reads it: its body swept over the fold's own
 *                  axes (Recomputed, src/Compiler/IR/terms.jl:70-86;
 *                  codegen/scalar.jl:88-110) */
enum { TH_TERM_LOAD = 0, TH_TERM_LIT = 1, TH_TERM_INDEX = 2, TH_TERM_STAT = 3, TH_TERM_APPLY = 4,
       TH_TERM_RECOMPUTE = 5 };

/* Functions, on fp32 (comparisons give 1 or 0; ifelse(c, a, b) takes a where
 * c != 0; round is to nearest, ties to even; max/min ignore a NaN operand). */
enum {
  TH_FN_ADD = 0, TH_FN_SUB, TH_FN_MUL, TH_FN_DIV, TH_FN_NEG, TH_FN_ABS, TH_FN_ABS2, TH_FN_SQRT,
  TH_FN_EXP, TH_FN_LOG, TH_FN_TANH, TH_FN_SIN, TH_FN_COS, TH_FN_LOG1P, TH_FN_EXPM1, TH_FN_POW,
  TH_FN_MAX, TH_FN_MIN, TH_FN_LT, TH_FN_LE, TH_FN_GT, TH_FN_GE, TH_FN_EQ, TH_FN_NE,
  TH_FN_IFELSE, TH_FN_ROUND, TH_FN_FLOOR, TH_FN_CEIL, TH_FN_SIGN, TH_FN_CLAMP, TH_FN_FMA,
  TH_FN_INV,
  TH_FN_BFLOAT16, /* x rounded to bfloat16 (nearest, ties to even) and widened back: Cast{BFloat16} */
  TH_FN_DROPOUT,  /* (key, position, rate): the dropout fixture's keep scale, 1 / (1 - rate) or 0, from
                     a wrapping 32-bit hash of the key and the 1-based position (stream 0);
                     test/fixtures/operations.jl:88-103 */
  TH_FN_COUNT
};

/* Folds (src/Compiler/IR/folds.jl:66-309), accumulating in fp32:
 *   TH_FOLD_SUM, _PROD, _MAX, _MIN  of the body
 *   TH_FOLD_EXP     Relative{Exponential}: the maximum m of the body y and
 *                   the sum of weight * exp(y - lse_shift(m)) (weight 1 when
 *                   the fold's weight is -1)
 *   TH_FOLD_SQUARE  Relative{Square}: the mean of the body and the sum of
 *                   squared deviations from it (Chan's combination)
 *   TH_FOLD_LINEAR  the linear recurrence h = a h' + b from h = 0, a the
 *                   body and b the weight: state (product of the a's, h),
 *                   combined earlier-first as (a2 a1, a2 b1 + b2) (the
 *                   `chain` of test/fixtures/programs.jl:54-55)
 *   TH_FOLD_ARGMAX, _ARGMIN  the extreme of the body and where it is, the
 *                   weight the element's index (required): state (y, i),
 *                   combined as Base's findmax (isless: NaN the largest,
 *                   -0.0 before 0.0) and findmin (isgreater: NaN the
 *                   smallest), the smaller index among equals (the `Better`
 *                   fold of src/Compiler/program/tracing.jl:735-790); indices
 *                   are exact to 2^24 */
enum { TH_FOLD_SUM = 0, TH_FOLD_PROD, TH_FOLD_MAX, TH_FOLD_MIN, TH_FOLD_EXP, TH_FOLD_SQUARE, TH_FOLD_LINEAR,
       TH_FOLD_ARGMAX, TH_FOLD_ARGMIN };

/* What a Stat term reads of a fold: the value (SUM, PROD, MAX, MIN; LINEAR:
 * h; ARGMAX, ARGMIN: the extreme); the statistic (EXP: m, SQUARE: the mean,
 * LINEAR: the product of the a's; ARGMAX, ARGMIN: its index); the sum (EXP: the weighted sum of exponentials, SQUARE: the squared
 * deviations); or, for EXP, the log-sum-exp lse_shift(m) + log(sum)
 * (LOGSUMEXP, folds.jl:263). */
enum { TH_OBSERVE_VALUE = 0, TH_OBSERVE_STATISTIC = 1, TH_OBSERVE_SUM = 2, TH_OBSERVE_LOGSUMEXP = 3 };

/* A Div or Mod atom: coeff * (inner div or mod divisor), inner = constant +
 * sum over k of inner[k] * i_k, with floor division and a remainder in
 * 0..divisor-1 (Div and Mod of IR/expressions.jl:24-34). */
enum { TH_PART_NONE = 0, TH_PART_DIV = 1, TH_PART_MOD = 2 };
typedef struct th_part {
  int32_t kind;       /* TH_PART_* */
  int32_t reserved;
  int64_t divisor;    /* > 0 */
  int64_t coeff;
  int64_t constant;
  int64_t inner[TH_FLOOR_RANK];
} th_part;

/* constant + sum over k of coeff[k] * i_k, the i_k the zero-based positions,
 * + the two parts (Div and Mod atoms, unused ones TH_PART_NONE),
 * + gather_coeff * (the value of term `gather`, a load of an integer value,
 * or of a float value holding integers, truncated)
 * when gather >= 0 (an Indirect atom; the atoms of IR/expressions.jl).  A
 * gathered address is clamped into its value on the device: an index out of
 * range reads or writes the nearest element instead of faulting. */
typedef struct th_affine {
  int64_t constant;
  int64_t coeff[TH_FLOOR_RANK];
  int32_t gather;
  int32_t reserved;
  int64_t gather_coeff;
  th_part part[2];
} th_affine;

typedef struct th_floor_value {
  int32_t dtype;    /* TH_F32 or TH_BF16; TH_I32 or TH_I64 for values only read (indices) */
  int32_t reserved;
  int64_t length;   /* elements */
  void* ptr;
} th_floor_value;

typedef struct th_term {
  int32_t op;       /* TH_TERM_* */
  int32_t fn;       /* TH_FN_*, for TH_TERM_APPLY */
  int32_t args[3];
  int32_t ref;      /* the value of a load, the fold of a statistic */
  int32_t observe;  /* TH_OBSERVE_*, for TH_TERM_STAT */
  float lit;
  th_affine index;  /* a load's element, an index term's expression */
} th_term;

typedef struct th_fold {
  int32_t kind;     /* TH_FOLD_* */
  int32_t phase;    /* >= 1; a fold's terms read statistics of earlier phases only
                       (in a scan group: of folds earlier in (phase, index) order);
                       0: a fold recomputed where a TH_TERM_RECOMPUTE reads it */
  int32_t body;     /* term */
  int32_t weight;   /* term, or -1; TH_FOLD_EXP, _LINEAR, _ARGMAX, _ARGMIN (required) only */
  int32_t scan;     /* scan groups: TH_SCAN_*; 0 elsewhere */
  int32_t n_inner;  /* phase 0: the axes it sweeps, 1..TH_FLOOR_RANK - rank */
  int64_t inner[TH_FLOOR_RANK]; /* their extents, positions rank, rank + 1, ... of
                                   the addresses of the terms its body reaches */
} th_fold;

/* A scan group's fold: its result after the sweep (a plain fold), or at each
 * position including (inclusive) or before (exclusive) the position's element. */
enum { TH_SCAN_NONE = 0, TH_SCAN_INCLUSIVE = 1, TH_SCAN_EXCLUSIVE = 2 };

/* Output: value[index(i)] = term, rounded to the value's type.  `full` outputs
 * are written at every position of the domain; the others once per item of a
 * reduction group, with the folded positions at zero (a fold's result stored
 * at its placement, or a statistic of it).  With `accumulate`, value[index(i)]
 * += term instead, atomically (fp32 values only): a fold by key whose
 * positions may repeat (accumulate!(::SumFold), ext/CUDAExt.jl:923-924); the
 * order of the additions, and so the last bits of a sum, may change run to run. */
typedef struct th_output {
  int32_t value;
  int32_t term;
  int32_t full;
  int32_t accumulate;
  th_affine index;
} th_output;

typedef struct th_floor_desc {
  int32_t kind;                       /* TH_GROUP_* */
  int32_t rank;                       /* 1..TH_FLOOR_RANK */
  int64_t extents[TH_FLOOR_RANK];
  uint32_t reduced;                   /* bit k: axis k is folded (scan groups: scanned) */
  int32_t n_values, n_terms, n_folds, n_outputs;
  int32_t flags;                      /* TH_FLOOR_REVERSE for a scan from the last position */
  const th_floor_value* values;
  const th_term* terms;               /* in order: args refer to earlier terms */
  const th_fold* folds;
  const th_output* outputs;
} th_floor_desc;

/* The group's launch.  Values: the group's values, in order.  Every address
 * the terms and outputs reach over the domain must lie inside its value. */
int th_build_floor(const th_floor_desc* desc, th_launch** host_out);

/* The generated source and how the group maps onto the device (a comment at
 * its head); needs no device.  *host_needed gets the size with the final NUL. */
int th_floor_source(const th_floor_desc* desc, char* host_out, size_t capacity, size_t* host_needed);

/* Generate and compile the group's kernels into the code-object cache,
 * without a device (the "does it build" check of a group).
 *
 * The cache is a directory of code objects (TEMPEST_HIP_CACHE, else
 * $XDG_CACHE_HOME/tempest_hip, else ~/.cache/tempest_hip), each named by a
 * hash of its generated source and the compiler options; the source names
 * the hiprtc and HIP runtime versions and the store's schema, so another
 * toolchain's entries are never read.  The store is bounded by
 * TEMPEST_HIP_CACHE_CAPACITY (bytes, or with a K/M/G suffix; 512 MiB by
 * default; 0 turns it off) and removes the entries used least recently.
 * Replaces the kernel store of src/Compiler/runtime/cache.jl:1-60 with its
 * bound JULIA_OBJCACHE_CAPACITY (:43-45). */
int th_floor_compile(const th_floor_desc* desc);

/* Code objects loaded from the store and compiled, in this process: the
 * counts cache_counts() reports, src/Compiler/runtime/cache.jl:56-58. */
int th_floor_cache_counts(int64_t* host_loaded, int64_t* host_compiled);

/* ---- the small program of config 1 -------------------------------------- */

/* loss(w, b, x) = sum(abs2, tanh.(w' * x .+ b)) and its gradient, one fused
 * kernel in one workgroup: w is d x h, b h, x d x c (Float32, column-major);
 * outputs loss (1), dw (d x h), db (h), dx (d x c).  p*(h + c) + h*c + 16
 * floats, p = d rounded up to 4 plus 4, must fit the workgroup's 64 KiB of LDS.
 * Values: 0 w, 1 b, 2 x, 3 loss, 4 dw, 5 db, 6 dx. */
int th_build_tanh_layer_grad(int32_t d, int32_t h, int32_t c,
                             const float* w, const float* b, const float* x,
                             float* loss, float* dw, float* db, float* dx,
                             th_launch** host_out);

/* ---- op class (b): bf16 products on the matrix cores --------------------- */

enum { TH_F32 = 0, TH_BF16 = 1, TH_I32 = 2, TH_I64 = 3, TH_F16 = 4 };

/* What the product's group fuses after it.  Every epilogue works on the fp32
 * accumulator and rounds once to bf16 where it stores, except where noted.
 *   TH_EPI_STORE          C = A*B (+ bias[i] if bias), bf16 or fp32.
 *   TH_EPI_GELU           Z = round(A*B + bias[i]) to C, H = gelu(Z) to aux_out
 *                         (tanh form, test/fixtures/programs.jl:19).
 *   TH_EPI_SQUARE_LOSS    y = round(A*B + bias[i]); loss = sum(y .^ 2) (fp32,
 *                         to *loss); C = dy = round(2y); row_sums[i] = the bf16
 *                         rounding of sum over j of dy[i, j] (the bias gradient).
 *   TH_EPI_GELU_BACKWARD  C = dz = round(round(A*B) .* gelu'(Z)), Z = aux
 *                         (bf16, m x n, column-major at aux_ld); row_sums[i] =
 *                         sum over j of dz[i, j], rounded to bf16. */
enum { TH_EPI_STORE = 0, TH_EPI_GELU = 1, TH_EPI_SQUARE_LOSS = 2, TH_EPI_GELU_BACKWARD = 3 };

/* C (m x n, column-major, leading dimension c_ld) = A (m x k) * B (k x n),
 * for each of `batch` products (C_z = D_z + A_z B_z with TH_GEMM_ACCUMULATE).
 * A's element (i, l) is a[i*a_m + l*a_k], B's (l, j) is b[l*b_k + j*b_n];
 * product z's operands start a_batch, b_batch, c_batch (d_batch) elements
 * further.  Factors are bf16 unless flags say fp32 or fp16; products
 * accumulate in fp32 and the result is rounded once.
 * Three implementations, by `tile`:
 *   TH_TILE_256: bf16 factors with a unit stride on each operand, m, n, k and
 *     the other strides multiples of 8, operands 16-byte aligned: 256 x 256
 *     tiles, every epilogue;
 *   TH_TILE_128X128, _128X64, _64X128, _64X64 (rows x columns of C): bf16 or
 *     fp16 factors with a unit stride on each operand, the other strides
 *     multiples of 8, operands 16-byte aligned, any m, n, k, TH_EPI_STORE
 *     (bias allowed), a result of the factors' type or fp32: the output tiles
 *     the reference's product sketch searches for half factors
 *     (ext/cuTileExt/contract.jl:36-39);
 *   TH_TILE_GENERAL: anything with TH_EPI_STORE and no bias, on the fp32
 *     matrix cores, any shape and strides: fp32 factors with an fp32 result on
 *     128 x 128 tiles (16-byte loads along a unit stride, K split like the
 *     others), half factors or a half result on 64 x 64 tiles (unsplit).
 *     fp32 factors run only here unless TH_GEMM_BF16X3.
 * TH_TILE_AUTO chooses: the 256 x 256 kernel where it takes the product and
 * fills the device (split or not), else the largest middle tile that gives
 * 256 workgroups (the smallest if none does), else the general kernel.
 * `splits` parts of K (256 and middle tiles, TH_EPI_STORE) are summed by a
 * second launch, with the bias and D; 0 chooses (parts when the tiles alone
 * would leave the device idle), 1 none.  th_gemm_tune measures the choices.
 * Values: 0 a, 1 b, 2 c, 3 bias, 4 aux, 5 aux_out, 6 row_sums, 7 loss, 8 d.
 * Replaces the cuTile product sketch (ext/cuTileExt/contract.jl:32-206) and
 * cuBLASProducts (ext/cuBLASExt.jl:23-36,247-259): its product, widened and
 * accumulated templates over a batch. */
typedef struct th_gemm_desc {
  int32_t m, n, k;
  int32_t c_dtype;   /* TH_BF16 or TH_F32 (TH_F32 only with TH_EPI_STORE) */
  int32_t epilogue;  /* TH_EPI_* */
  int32_t tile;      /* TH_TILE_*: which kernel and output tile */
  const void* a;
  int64_t a_m, a_k;
  const void* b;
  int64_t b_k, b_n;
  void* c;
  int64_t c_ld;
  const void* bias;  /* bf16, m */
  const void* aux;   /* bf16 */
  int64_t aux_ld;
  void* aux_out;     /* bf16, C's layout */
  void* row_sums;    /* bf16, m */
  float* loss;       /* fp32, one */
  int32_t batch;     /* products (0 or 1: one) */
  int32_t flags;     /* TH_GEMM_* */
  int64_t a_batch, b_batch, c_batch;
  const void* d;     /* TH_GEMM_ACCUMULATE: C = D + A*B, D laid out as C, may be C itself */
  int64_t d_ld, d_batch;  /* 0, 0: C's */
  int32_t splits;    /* parts K is split into: 0 chosen, 1 none */
  int32_t reserved2;
} th_gemm_desc;

#define TH_GEMM_F32_FACTORS 1  /* a and b hold fp32 */
#define TH_GEMM_F16_FACTORS 2  /* a and b hold fp16 */
#define TH_GEMM_ACCUMULATE 4   /* C = D + A*B (cuBLASExt.jl:25, `accumulated`) */
/* With TH_GEMM_F32_FACTORS: each fp32 factor split x = hi + lo in bf16
 * (hi = bf16(x), lo = bf16(x - hi)) and the product run on the bf16 tile
 * kernels as A_hi B_hi + A_hi B_lo + A_lo B_hi, summed in fp32 (one product
 * over K tripled; the tripled operands in the launch's workspace): about 16
 * of fp32's 24 significant bits, on matrix cores 16x faster than fp32's.
 * The MI355X counterpart of the reference's precision = :tf32x3
 * (src/Compiler/runtime/target.jl:42-44, ext/cuBLASExt.jl:61-65).  An fp32
 * result, no epilogue or bias; tile AUTO or one of the bf16 tiles. */
#define TH_GEMM_BF16X3 8

#define TH_TILE_AUTO 0
#define TH_TILE_256 1
#define TH_TILE_128X128 2
#define TH_TILE_128X64 3
#define TH_TILE_64X128 4
#define TH_TILE_64X64 5
#define TH_TILE_GENERAL 6

int th_build_gemm(const th_gemm_desc* desc, th_launch** host_out);

/* Measure the product's choices on the device and return the fastest: its
 * tile (TH_TILE_*), its parts of K and its time (seconds, as
 * th_time_launch measures).  The search runs in stages as the reference's
 * cover searches a product's tiles (ext/cuTileExt/contract.jl:12-27,171-200,
 * tinygrad's beam search at width one): every tile that takes the product at
 * its chosen split, then the other splits (1, 2, 4, ... 16, each part at
 * least 256 deep) of the best.  `desc`'s tile and splits are ignored; its
 * arrays are the ones measured on, and the product's outputs (c, and what
 * the epilogue writes) are overwritten; D + A B in place (d == c) is refused.
 * Results are kept for the process, keyed by the product's shape, layouts,
 * types and epilogue, so a second call measures nothing. */
int th_gemm_tune(const th_gemm_desc* desc, int32_t* tile_out, int32_t* splits_out, double* seconds_out);

/* Products alike but for where their operands start, as one launch: each of
 * descs[0..count) built as th_build_gemm builds it, run in order.  Value v of
 * product i is value 9 i + v of the launch.  Replaces cuBLASProducts' build
 * over a vector of bindings (cublasGemmBatchedEx on arrays of addresses,
 * ext/cuBLASExt.jl:262-326). */
int th_build_gemm_grouped(const th_gemm_desc* descs, int count, th_launch** host_out);

/* ---- op class (c): causal flash attention ------------------------------- */

/* Attention over (features, heads, positions, batch) column-major arrays
 * (test/fixtures/operations.jl:5-70): element (d, h, s, b) of q, o, dout, dq
 * at d + h*q_strides[0] + s*q_strides[1] + b*q_strides[2], of k, v, dk, dv at
 * d + h*k_strides[0] + s*k_strides[1] + b*k_strides[2]; query head h reads
 * key/value head h / (heads / kv_heads).  lse is fp32, (1, heads, positions,
 * batch): element (h, s, b) at h + heads*(s + seq*b), the natural log-sum-exp
 * of each query's scaled scores.  scale <= 0 means 1/sqrt(head_dim).
 * Two implementations: bf16 with head_dim 128, seq a multiple of 128, keys
 * as many as queries and no device-held masks runs the matrix-core kernels;
 * anything else with head_dim 1..256 (fp32 or bf16 arrays, any lengths,
 * starts and lengths masks) runs the general kernels, which compute in fp32
 * on the vector ALUs (the cuDNN claim's d <= 256, ext/cuDNNExt.jl:95-100, and
 * the reference's attention tests, test/cuda/attention.jl:10-16,218-271). */
typedef struct th_attention_desc {
  int32_t batch, heads, kv_heads, seq, head_dim;
  int32_t causal;
  float scale;
  int32_t flags; /* TH_ATTN_F32; backward: TH_ATTN_RECOMPUTE_DQ */
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  const void* dout;
  void* dq;
  void* dk;
  void* dv;
  int64_t q_strides[3]; /* along heads, positions, batch */
  int64_t k_strides[3];
  int32_t kv_seq;         /* positions of k and v; 0: the same as seq */
  int32_t reserved;
  /* Masks the device holds (NULL: none), read when the launch runs:
   * starts, int32 (positions, batch): the 1-based first key query (s, b)
   * sees, at s + seq * b (documents packed in sequences);
   * lengths, int32 (batch): the keys sequence b holds (decode over a cache).
   * Query j (0-based) of batch b sees key i when i < lengths[b],
   * i >= starts[j + seq b] - 1 and, causal, i <= j. */
  const int32_t* starts;
  const int32_t* lengths;
} th_attention_desc;

/* q, k, v, o, dout, dq, dk, dv hold fp32 instead of bf16. */
#define TH_ATTN_F32 2

/* o = softmax(scale * k'q, masked) * v per head, and lse (if non-NULL).
 * Values: 0 q, 1 k, 2 v, 3 o, 4 lse, 5 starts, 6 lengths.  Replaces the cuTile online-softmax
 * product sweep (ext/cuTileExt/build.jl:326-532) and cuDNNAttention's SDPA
 * forward (ext/cuDNNExt.jl:38-55,116-210). */
int th_build_attention_fwd(const th_attention_desc* desc, th_launch** host_out);

/* Backward flag: never store dS; the dQ sweep recomputes S and dP instead. */
#define TH_ATTN_RECOMPUTE_DQ 1

/* dq, dk, dv from q, k, v, o, lse (as the forward wrote them) and dout;
 * deterministic (no atomics); the general kernels need lse.  With grouped heads (kv_heads < heads) dk and
 * dv sum over the heads / kv_heads query heads that read each key/value
 * head, swept in turn (test/cuda/attention.jl:132-140).  The dK/dV sweep stores dS
 * (bf16, 2*batch*heads*seq^2 bytes of the launch's workspace, th_launch_workspace)
 * for the dQ sweep; when that exceeds 16 GiB, or with TH_ATTN_RECOMPUTE_DQ, the
 * dQ sweep recomputes S and dP instead and the workspace holds only the row
 * statistics.
 * Values: 0 q, 1 k, 2 v, 3 o, 4 lse, 5 dout, 6 dq, 7 dk, 8 dv, 9 starts,
 * 10 lengths.  Replaces the
 * cuTile transposed folds of the backward (ext/cuTileExt/transpose.jl:1-213). */
int th_build_attention_bwd(const th_attention_desc* desc, th_launch** host_out);

/* ---- config 5: chunked gated DeltaNet (scan + recurrence) ---------------- */

/* The gated delta rule per (batch, head) sequence, S (dk x dv) from zero:
 *   S = exp(a_t) (I - beta_t k_t k_t') S + beta_t k_t v_t',  o_t = S' q_t
 * (examples/deltanet.jl:89-101), computed in chunks of 64 positions as
 * examples/deltanet.jl:58-86 writes it.  q, k, v, o, dout, dq, dk_out, dv_out
 * are bf16 (d, heads, positions, batch): element (d, h, t, b) at
 * d + h*strides[0] + t*strides[1] + b*strides[2]; a (the log-gates) and beta,
 * da, dbeta are fp32 (heads, positions, batch) at gate_strides.  dk = dv =
 * 128, chunk 64, seq a multiple of 64.  The gradient is of
 * sum(o .* dout) with respect to q, k, v, a and beta; there o may be null, and
 * is then kept in the launch's workspace (laid out at q's strides).  The chunk
 * intermediates lie in the workspace (th_launch_workspace).
 * Values: 0 q, 1 k, 2 v, 3 a, 4 beta, 5 o, 6 dout, 7 dq, 8 dk, 9 dv, 10 da,
 * 11 dbeta.  Replaces the scan and recurrence sketches (ext/cuTileExt/
 * build.jl:715-839; codegen/scalar.jl:354-440; runtime/stepped.jl). */
typedef struct th_deltanet_desc {
  int32_t batch, heads, seq, dk, dv, chunk;
  const void* q;
  const void* k;
  const void* v;
  const float* a;
  const float* beta;
  void* o;
  const void* dout;
  void* dq;
  void* dk_out;
  void* dv_out;
  float* da;
  float* dbeta;
  int64_t strides[3];      /* along heads, positions, batch */
  int64_t gate_strides[3]; /* along heads, positions, batch */
} th_deltanet_desc;

/* The forward alone (o). */
int th_build_deltanet_fwd(const th_deltanet_desc* desc, th_launch** host_out);

/* The forward and the gradient (o, dq, dk, dv, da, dbeta) in one launch. */
int th_build_deltanet(const th_deltanet_desc* desc, th_launch** host_out);

#ifdef __cplusplus
}
#endif

#endif /* TEMPEST_HIP_H */
