// Internal core of libtempest_hip: the launch object every builder returns,
// error reporting, and the helpers kernels share.  Not part of the ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/tempest_hip.h"

namespace th {

// ---- errors --------------------------------------------------------------

void set_error(const std::string& message);
int fail(int code, const std::string& message);
int hip_fail(hipError_t e, const char* what);

#define TH_HIP(call)                                   \
  do {                                                 \
    hipError_t th_e_ = (call);                         \
    if (th_e_ != hipSuccess) return ::th::hip_fail(th_e_, #call); \
  } while (0)

#define TH_REQUIRE(cond, msg)                                      \
  do {                                                             \
    if (!(cond)) return ::th::fail(TH_E_ARGUMENT, (msg));          \
  } while (0)

// ---- context ---------------------------------------------------------------

struct Context {
  bool ready = false;
  int device = -1;
  hipStream_t own = nullptr;     // the library's stream (default priority)
  hipStream_t stream = nullptr;  // where launches go: `own` or the caller's
  hipDeviceProp_t prop{};
  // Cache clearing for timings: a buffer of 2 x (L2 + MALL) read through.
  void* clear_buf = nullptr;
  size_t clear_bytes = 0;
  uint32_t* sink = nullptr;
  double replay_overhead = -1.0;
  double launch_gap = -1.0;  // seconds a launch takes inside a long replayed graph
  double graph_base = -1.0;  // seconds a replay costs beyond its launches, back to back
  double cached_rate = -1.0;  // bytes/s read from what L2 + MALL hold
  double direct_gap = -1.0;  // seconds a direct launch of an empty kernel takes, back to back
};

Context& ctx();
int require_ready();

// ---- launches --------------------------------------------------------------

// One kernel of a launch: the function, its grid, and its single by-value
// argument struct, kept as bytes so that values can be repointed in place.
struct Kernel {
  const void* fn = nullptr;
  // A kernel compiled at run time (the generated floor): its module function,
  // launched through the module API; `fn` is then null.
  hipFunction_t module = nullptr;
  const char* name = "";
  dim3 grid{1, 1, 1};
  dim3 block{1, 1, 1};
  uint32_t shmem = 0;
  alignas(16) unsigned char args[512];
  uint32_t args_size = 0;
};

// Where a value's address lives: a kernel of the launch and a byte offset
// into that kernel's argument struct.
struct Ref {
  int kernel;
  uint32_t offset;
};

// A pointer into the launch's workspace: kernel, byte offset of the pointer
// in its arguments, byte offset of what it points at in the workspace.
struct WsRef {
  int kernel;
  uint32_t offset;
  uint64_t at;
};

}  // namespace th

struct th_launch {
  std::string name;
  std::vector<th::Kernel> kernels;
  std::vector<std::vector<th::Ref>> values;  // per value: every place it is read
  std::vector<uint32_t> align;               // per value: the alignment the build assumed
  std::vector<void*> owned;                  // buffers the launch owns
  // The workspace: device memory its kernels use beyond its values, given by
  // the caller (th_launch_set_workspace) or allocated at the first run or
  // capture, then owned.
  uint64_t ws_bytes = 0;
  void* ws = nullptr;
  bool ws_owned = false;
  std::vector<th::WsRef> ws_refs;
  th_work work{};
};

namespace th {

// A launch under construction: kernels added with their argument struct,
// value references by member offset.
class Builder {
 public:
  explicit Builder(const char* name, int values) {
    l_ = new th_launch();
    l_->name = name;
    l_->values.resize(values);
    l_->align.assign(values, 4);
  }
  ~Builder() { delete l_; }

  template <class Args>
  int kernel(const void* fn, const char* name, dim3 grid, dim3 block, uint32_t shmem,
             const Args& a) {
    static_assert(sizeof(Args) <= sizeof(Kernel::args), "kernel argument struct too large");
    Kernel k;
    k.fn = fn;
    k.name = name;
    k.grid = grid;
    k.block = block;
    k.shmem = shmem;
    std::memcpy(k.args, &a, sizeof(Args));
    k.args_size = sizeof(Args);
    l_->kernels.push_back(k);
    return static_cast<int>(l_->kernels.size()) - 1;
  }
  // Value `v` is the pointer at byte `offset` of kernel `k`'s arguments.
  void ref(int v, int k, size_t offset) { l_->values[v].push_back(Ref{k, (uint32_t)offset}); }
  // Value `v` must stay aligned to `bytes` when it is repointed.
  void align(int v, uint32_t bytes) { l_->align[v] = std::max(l_->align[v], bytes); }
  void own(void* p) { l_->owned.push_back(p); }
  // Reserve `bytes` of the launch's workspace (256-byte aligned pieces, laid
  // out in order); returns the piece's offset in it.
  uint64_t workspace(uint64_t bytes) {
    const uint64_t at = l_->ws_bytes;
    l_->ws_bytes += (std::max<uint64_t>(bytes, 1) + 255) / 256 * 256;
    return at;
  }
  // The pointer at byte `offset` of kernel `k`'s arguments is workspace + at.
  void ws_ref(int k, size_t offset, uint64_t at) { l_->ws_refs.push_back(WsRef{k, (uint32_t)offset, at}); }
  // A kernel compiled at run time: `fn` is a module function.
  template <class Args>
  int module_kernel(hipFunction_t fn, const char* name, dim3 grid, dim3 block, uint32_t shmem,
                    const Args& a, size_t bytes) {
    static_assert(sizeof(Args) <= sizeof(Kernel::args), "kernel argument struct too large");
    Kernel k;
    k.module = fn;
    k.name = name;
    k.grid = grid;
    k.block = block;
    k.shmem = shmem;
    std::memcpy(k.args, &a, bytes);
    k.args_size = (uint32_t)bytes;
    l_->kernels.push_back(k);
    return static_cast<int>(l_->kernels.size()) - 1;
  }
  void work(double bytes, double flops, int64_t blocks) {
    l_->work.bytes = bytes;
    l_->work.flops = flops;
    l_->work.blocks = blocks;
  }
  th_launch* release() {
    l_->work.kernels = (int32_t)l_->kernels.size();
    l_->work.values = (int32_t)l_->values.size();
    th_launch* out = l_;
    l_ = nullptr;
    return out;
  }

 private:
  th_launch* l_;
};

#define TH_OFFSET(Args, member) offsetof(Args, member)

int launch_kernel(const Kernel& k, hipStream_t s);
// Give the launch its workspace if it has none yet (allocated and owned).
int ensure_workspace(th_launch* l);
// Write the workspace's address into the kernel arguments that use it.
void point_workspace(th_launch* l);
// Find, on `device` (current), the address of the static scratch that
// th_softmax_grad_noalloc uses; th_init calls it once per device.
int rows_scratch_setup(int device);
int device_alloc(size_t bytes, void** out);

// The parts an attention sweep of `length` positions takes when `groups`
// workgroups (unsplit, unpaired) would leave the device idle: enough for
// about 512 workgroups where they are fewer than 256 (one a CU), at most 8,
// each at least 128 positions (span, a multiple of 64).  Each wave's sweep
// bounds a small grid; parts share it among more waves, at the cost of
// fp32 partial results and a launch that adds them.
struct Split {
  int n, span;
};
inline Split split_of(int64_t groups, int length) {
  if (groups >= 256 || length <= 128) return {1, 0};
  int n = (int)std::min<int64_t>(8, (512 + groups - 1) / groups);
  n = std::min(n, (length + 127) / 128);
  if (n <= 1) return {1, 0};
  const int span = ((length + n - 1) / n + 63) / 64 * 64;
  return {(length + span - 1) / span, span};
}

// Attention for what the matrix-core kernels do not take (attention_generic.hip).
int build_attention_general_fwd(const th_attention_desc* d, th_launch** out);
int build_attention_general_bwd(const th_attention_desc* d, th_launch** out);
// Attention on the matrix cores at head dims 64, 128 and 256 and any lengths
// (attention_mfma.hip): what the tuned kernels do not take, bf16, no masks.
bool mfma_attention_takes(const th_attention_desc* d);
int build_attention_mfma_fwd(const th_attention_desc* d, th_launch** out);
int build_attention_mfma_bwd(const th_attention_desc* d, th_launch** out);
// fp32 arrays on the matrix cores (attention_f32.hip): head dims 64 and 128,
// no device-held masks.
bool f32_attention_takes(const th_attention_desc* d);
int build_attention_f32_fwd(const th_attention_desc* d, th_launch** out);
int build_attention_f32_bwd(const th_attention_desc* d, th_launch** out);
// Products the bf16 tile kernel does not take (gemm_general.hip).
int build_gemm_general(const th_gemm_desc* d, th_launch** out);

}  // namespace th

// ---- device helpers shared by kernels ---------------------------------------

namespace thd {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// x[0] + x[stride] + ... + x[(n - 1) stride] (T a float or a float vector,
// stride in elements of T), added in that order, the loads issued eight at a
// time: a loop of one load and its add waits a memory round trip per term.
template <class T>
__device__ __forceinline__ T sum_in_order(const T* x, int64_t stride, int n) {
  T s = {};
  int k = 0;
  for (; k + 8 <= n; k += 8) {
    T v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = x[(int64_t)(k + u) * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; k < n; ++k) s += x[(int64_t)k * stride];
  return s;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// The shift an exponential sum takes against maximum m: m itself when finite,
// zero otherwise, so that an empty or all -Inf run sums to zero
// (lse_shift, src/Compiler/IR/folds.jl:194).
__device__ __forceinline__ float lse_shift(float m) { return isfinite(m) ? m : 0.0f; }

}  // namespace thd
