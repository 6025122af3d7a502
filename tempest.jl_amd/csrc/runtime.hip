// libtempest_hip runtime: errors, device and stream, storage (buffers and the
// slot arena), launch objects, graphs and timing.  The Target protocol of the
// reference (src/Compiler/runtime/target.jl) as a C ABI for one gfx950 GPU.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "th_core.h"

namespace th {

// ---- errors ----------------------------------------------------------------

static thread_local std::string g_error;

void set_error(const std::string& message) { g_error = message; }

int fail(int code, const std::string& message) {
  g_error = message;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  g_error = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
  return static_cast<int>(e);
}

// ---- context ---------------------------------------------------------------

static Context g_ctx;
static std::mutex g_timing;  // timings run one at a time (target.jl:619-628)

Context& ctx() { return g_ctx; }

int require_ready() {
  if (!g_ctx.ready) return fail(TH_E_STATE, "libtempest_hip: th_init has not been called");
  return TH_OK;
}

int device_alloc(size_t bytes, void** out) {
  *out = nullptr;
  if (bytes == 0) bytes = 256;
  hipError_t e = hipMalloc(out, bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(TH_E_MEMORY, std::string("hipMalloc of ") + std::to_string(bytes) +
                                 " bytes failed: " + hipGetErrorString(e));
  }
  return TH_OK;
}

// Write the workspace's address into every kernel argument that points into it.
void point_workspace(th_launch* l) {
  for (const WsRef& r : l->ws_refs) {
    void* at = static_cast<char*>(l->ws) + r.at;
    std::memcpy(l->kernels[r.kernel].args + r.offset, &at, sizeof(void*));
  }
}

int ensure_workspace(th_launch* l) {
  if (l->ws_bytes == 0 || l->ws) return TH_OK;
  if (int r = device_alloc(l->ws_bytes, &l->ws)) return r;
  l->ws_owned = true;
  point_workspace(l);
  return TH_OK;
}

int launch_kernel(const Kernel& k, hipStream_t s) {
  void* params[1] = {const_cast<unsigned char*>(k.args)};
  hipError_t e = k.module
                     ? hipModuleLaunchKernel(k.module, k.grid.x, k.grid.y, k.grid.z, k.block.x, k.block.y,
                                             k.block.z, k.shmem, s, params, nullptr)
                     : hipLaunchKernel(k.fn, k.grid, k.block, params, k.shmem, s);
  if (e != hipSuccess) return hip_fail(e, k.name);
  return TH_OK;
}

}  // namespace th

namespace th {
// Timing helpers (below): the cache-clearing buffer, what a replay adds, and
// the rate of reads the caches serve.
static int ensure_clearing();
static int replay_overhead(double* out);
static int cached_rate(double* out);
}  // namespace th

using namespace th;

// A kernel that does nothing: what a replay alone adds is timed with it.
__global__ void th_blank_kernel(int) {}

// Read `words` 32-bit words, keeping their xor only where zeros could not give
// it, so that the reads stay: the cache clearing of a timing
// (read_through, ext/CUDAExt.jl:837-850).  Ordinary loads, which allocate in
// L2 and in the Infinity Cache (MALL), so that reading twice their size
// evicts both; non-temporal loads left the MALL holding what a timed launch
// read before (a 16 MB column sum then measured 16 TB/s).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
struct ClearArgs {
  const u32x4* a;
  uint32_t* sink;
  uint64_t n;
  int passes;  // reads of the n words, one after another
};
__global__ __launch_bounds__(256) void th_clear_kernel(ClearArgs c) {
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint32_t s = 0;
  for (int p = 0; p < c.passes; ++p)
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < c.n; i += stride) {
      u32x4 v = c.a[i];
      s ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
  if (s == 0xffffffffu) c.sink[0] = s;
}


// A copy of `bytes` bytes as a kernel, so that a graph records it beside the
// launches and retargets it as one (the reference's `Copy` step,
// src/Compiler/runtime/runtime.jl:47-64).  16-byte words where both ends and
// the length allow, bytes otherwise: the choice is made per launch from the
// addresses it holds, so any repointing keeps it correct.
struct CopyArgs {
  unsigned char* dst;
  const unsigned char* src;
  uint64_t bytes;
};
__global__ __launch_bounds__(256) void th_copy_kernel(CopyArgs c) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if ((((uintptr_t)c.dst | (uintptr_t)c.src | c.bytes) & 15) == 0) {
    u32x4* d = reinterpret_cast<u32x4*>(c.dst);
    const u32x4* s = reinterpret_cast<const u32x4*>(c.src);
    for (uint64_t i = t; i < c.bytes / 16; i += stride) d[i] = __builtin_nontemporal_load(s + i);
  } else {
    for (uint64_t i = t; i < c.bytes; i += stride) c.dst[i] = c.src[i];
  }
}


// ---- the matrix cores' sustained rate ---------------------------------------------------
// Every SIMD of the device runs two waves of back-to-back
// v_mfma_f32_32x32x16_bf16 on operands held in registers (four independent
// accumulators a wave): with one operand pair throughout, or with eight
// pairs of random bits cycled so that every product's operands differ from
// the last one's, as a real product's do.  Each wave reads the shader clock
// counter and the 100 MHz real-time counter at its start and end, so the run
// reports the clock the matrix cores actually ran at.
typedef __bf16 th_bf16x8 __attribute__((ext_vector_type(8)));
typedef float th_f32x16 __attribute__((ext_vector_type(16)));

struct RateArgs {
  const u32x4* seed;   // 8 operand pairs' bits per lane
  float* sink;         // written only if the sums come out as a value they never do
  uint64_t* stamps;    // per workgroup: clock start, end, real-time start, end
  int32_t iters;
  int32_t vary;
};

__global__ __launch_bounds__(256, 2) void th_matrix_rate_kernel(RateArgs a) {
  const int lane = threadIdx.x % 64;
  th_bf16x8 A[8], B[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    A[s] = __builtin_bit_cast(th_bf16x8, a.seed[(2 * s) * 64 + lane]);
    B[s] = __builtin_bit_cast(th_bf16x8, a.seed[(2 * s + 1) * 64 + lane]);
  }
  th_f32x16 acc[4] = {th_f32x16{}, th_f32x16{}, th_f32x16{}, th_f32x16{}};
  const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < a.iters; ++it) {
    if (a.vary) {
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[s], B[(s + j) % 8], acc[j], 0, 0, 0);
    } else {
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[0], B[0], acc[j], 0, 0, 0);
    }
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float x = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) x += acc[j][0] + acc[j][15];
  if (x == 1234.5f) a.sink[blockIdx.x] = x;
  if (threadIdx.x == 0) {
    a.stamps[4 * blockIdx.x + 0] = t0;
    a.stamps[4 * blockIdx.x + 1] = t1;
    a.stamps[4 * blockIdx.x + 2] = r0;
    a.stamps[4 * blockIdx.x + 3] = r1;
  }
}

// ---- the LDS read rate --------------------------------------------------------------
// Workgroups of four waves read a 64 KB LDS array in a loop, eight reads in
// flight a wave, at conflict-free addresses (each wave a different 8 KB
// block per read): ds_read_b128 (modes 0 and 2) or pairs of
// ds_read_b64_tr_b16 (modes 1 and 3), 16 bytes a lane either way.  Modes 2
// and 3 also issue one v_mfma_f32_32x32x16_bf16 on each 1 KB read, 32 flops
// a byte: the ratio of the attention sweeps' products to their fragment
// reads.  Clock and real-time stamps as in the matrix-rate kernel.
typedef short th_s16x4 __attribute__((ext_vector_type(4)));
typedef short th_s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) th_s16x4 th_lds_s16x4;

struct LdsRateArgs {
  uint32_t* sink;     // written only if the reads fold to a value they never do
  uint64_t* stamps;   // per workgroup: clock start, end, real-time start, end
  int32_t iters;
};

template <int kMode>
__global__ __launch_bounds__(256, 2) void th_lds_rate_kernel(LdsRateArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[32768];
  for (int i = threadIdx.x; i < 32768; i += 256) lds[i] = (uint16_t)(i * 7 + 1);
  __syncthreads();
  const int lane = threadIdx.x % 64, w = threadIdx.x / 64;
  u32x4 x = {0, 0, 0, 0};
  th_f32x16 acc[2] = {th_f32x16{}, th_f32x16{}};
  const th_bf16x8 b = __builtin_bit_cast(th_bf16x8, u32x4{0x3f803f80u ^ (uint32_t)lane, 0x3f803f81u, 0x3f803f82u, 0x3f803f83u});
  const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < a.iters; ++it) {
    asm volatile("" ::: "memory");  // read the array again every iteration
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int base = ((u + 2 * w) & 7) * 4096;
      u32x4 r;
      if constexpr (kMode == 0 || kMode == 2) {
        r = *reinterpret_cast<const u32x4*>(lds + base + 8 * lane);
      } else {
        const th_s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((th_lds_s16x4*)(lds + base + 4 * lane));
        const th_s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((th_lds_s16x4*)(lds + base + 256 + 4 * lane));
        r = __builtin_bit_cast(u32x4, th_s16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
      }
      x ^= r;
      if constexpr (kMode >= 2)
        acc[u & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(th_bf16x8, r), b, acc[u & 1], 0, 0, 0);
    }
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  const uint32_t y = x[0] ^ x[1] ^ x[2] ^ x[3] ^ __float_as_uint(acc[0][0] + acc[1][3]);
  if (y == 0x12345678u) a.sink[blockIdx.x] = y;
  if (threadIdx.x == 0) {
    a.stamps[4 * blockIdx.x + 0] = t0;
    a.stamps[4 * blockIdx.x + 1] = t1;
    a.stamps[4 * blockIdx.x + 2] = r0;
    a.stamps[4 * blockIdx.x + 3] = r1;
  }
}

// ---- the HBM read rate -------------------------------------------------------------
// Waves stream 1 KB wave loads (16 bytes a lane, non-temporal) from a device
// buffer, eight in flight, one workgroup of four waves a CU (96 KB of LDS
// requested and unused to hold it there).  Mode 0: each of 4 waves x CUs
// streams its own contiguous 2 MB.  Mode 1: the attention dQ sweep's dS'
// reads at B 8, H 16, S 4096 (a 4 GiB array): per (batch, head) 64 streams of
// 512 KB (64-query blocks); workgroup x of a (head, batch) takes 256-query
// blocks x and 15 - x, wave w streaming block 4 qb + w over steps 0 ..
// 4 qb + 3 of 8 KB, clamped to its own diagonal (step q64), the workgroups in
// XCD-contiguous order.  Every address lies inside the array.
struct ReadRateArgs {
  const u32x4* src;
  uint32_t* sink;  // written only if the reads fold to a value they never do
  int32_t mode;
};

__global__ __launch_bounds__(256) void th_read_rate_kernel(ReadRateArgs a) {
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  uint32_t x = 0;
  auto consume = [&](const u32x4* q) {
    u32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = __builtin_nontemporal_load(q + 64 * u);
#pragma unroll
    for (int u = 0; u < 8; ++u) x ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  };
  if (a.mode == 0) {
    const int64_t per = (int64_t)2 * 1024 * 1024 / 16;  // 16-byte units a wave
    const u32x4* q = a.src + ((int64_t)blockIdx.x * 4 + wave) * per + lane;
    for (int64_t i = 0; i < per; i += 512) consume(q + i);
  } else {
    const int S = 4096, H = 16, nq64 = S / 64, nqb = S / 256;
    int t = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    const int total = gridDim.x * gridDim.y * gridDim.z;
    t = (t % 8) * (total / 8) + t / 8;
    const int bx = t % gridDim.x, h = (t / gridDim.x) % gridDim.y, b = t / (gridDim.x * gridDim.y);
    for (int pass = 0; pass < 2; ++pass) {
      const int qb = pass == 0 ? bx : nqb - 1 - bx;
      const int q64 = 4 * qb + wave;
      const u32x4* q = a.src + (((int64_t)b * H + h) * nq64 + q64) * ((int64_t)S * 64 * 2 / 16) + lane;
      for (int kb = 0; kb < 4 * qb + 4; ++kb) consume(q + (int64_t)min(kb, q64) * 512);
    }
  }
  if (x == 0x12345678u) a.sink[blockIdx.x] = x;
}

extern "C" {

const char* th_last_error(void) { return g_error.c_str(); }

int th_init(int device) {
  Context& c = ctx();
  if (c.ready) {
    if (c.device == device) return TH_OK;
    return fail(TH_E_STATE, "libtempest_hip drives one device per process; already on device " +
                                std::to_string(c.device));
  }
  int count = 0;
  TH_HIP(hipGetDeviceCount(&count));
  if (device < 0 || device >= count)
    return fail(TH_E_ARGUMENT, "no device " + std::to_string(device) + " (" +
                                   std::to_string(count) + " visible)");
  TH_HIP(hipSetDevice(device));
  TH_HIP(hipGetDeviceProperties(&c.prop, device));
  TH_HIP(hipStreamCreateWithFlags(&c.own, hipStreamNonBlocking));
  if (int r = rows_scratch_setup(device)) return r;
  c.stream = c.own;
  c.device = device;
  c.ready = true;
  return TH_OK;
}

int th_shutdown(void) {
  Context& c = ctx();
  if (!c.ready) return TH_OK;
  TH_HIP(hipDeviceSynchronize());
  if (c.clear_buf) TH_HIP(hipFree(c.clear_buf));
  if (c.sink) TH_HIP(hipFree(c.sink));
  if (c.own) TH_HIP(hipStreamDestroy(c.own));
  c = Context{};
  return TH_OK;
}

int th_device_name(char* out, size_t capacity) {
  if (int r = require_ready()) return r;
  const hipDeviceProp_t& p = ctx().prop;
  std::snprintf(out, capacity, "%s (%s)", p.name, p.gcnArchName);
  return TH_OK;
}

int th_toolchain(char* out, size_t capacity) {
  int rt = 0;
  (void)hipRuntimeGetVersion(&rt);
  std::snprintf(out, capacity, "hip=%d;clang=%s;arch=gfx950", rt, __clang_version__);
  return TH_OK;
}

int th_device_rates(th_rates* out) {
  if (int r = require_ready()) return r;
  const hipDeviceProp_t& p = ctx().prop;
  int clock_khz = 0, bus_bits = 0;
  TH_HIP(hipDeviceGetAttribute(&clock_khz, hipDeviceAttributeMemoryClockRate, ctx().device));
  TH_HIP(hipDeviceGetAttribute(&bus_bits, hipDeviceAttributeMemoryBusWidth, ctx().device));
  // HBM3E as the runtime reports it on MI355X: a 2 GHz memory clock, four
  // transfers a clock on each of 8192 pins (8 Gb/s a pin, 8.2 TB/s);
  // bytes/s = 4 * clock * pins / 8.
  double bandwidth = 4.0 * 1.0e3 * clock_khz * bus_bits / 8.0;
  // CDNA4 has 256 MiB of MALL (Infinity Cache) behind the XCDs' L2.
  double cache = (double)p.l2CacheSize + 256.0 * 1024 * 1024;
  // The launch gap and the cached read rate measured on this device, once
  // per process.
  double cached = 0;
  {
    std::lock_guard<std::mutex> lock(g_timing);
    if (int r = ensure_clearing()) return r;
    double overhead = 0;
    if (int r = replay_overhead(&overhead)) return r;
    if (int r = cached_rate(&cached)) return r;
  }
  out->launch = ctx().launch_gap;
  out->bandwidth = bandwidth;
  out->cached = cached;
  out->cache = cache;
  out->blocks = (double)p.multiProcessorCount;
  return TH_OK;
}

int th_set_stream(void* stream) {
  if (int r = require_ready()) return r;
  ctx().stream = static_cast<hipStream_t>(stream);
  return TH_OK;
}

int th_get_stream(void** out) {
  if (int r = require_ready()) return r;
  *out = ctx().stream;
  return TH_OK;
}

int th_quiesce(void) {
  if (int r = require_ready()) return r;
  TH_HIP(hipStreamSynchronize(ctx().stream));
  return TH_OK;
}

// ---- storage ---------------------------------------------------------------

int th_alloc(size_t bytes, void** out) {
  if (int r = require_ready()) return r;
  return device_alloc(bytes, out);
}

int th_free(void* ptr) {
  if (int r = require_ready()) return r;
  if (ptr) TH_HIP(hipFree(ptr));
  return TH_OK;
}

int th_upload(void* dst, const void* src, size_t bytes) {
  if (int r = require_ready()) return r;
  if (bytes == 0) return TH_OK;
  TH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx().stream));
  // The host array may be freed once the call returns.
  TH_HIP(hipStreamSynchronize(ctx().stream));
  return TH_OK;
}

int th_download(void* dst, const void* src, size_t bytes) {
  if (int r = require_ready()) return r;
  if (bytes == 0) return TH_OK;
  TH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx().stream));
  TH_HIP(hipStreamSynchronize(ctx().stream));
  return TH_OK;
}

int th_copy(void* dst, const void* src, size_t bytes) {
  if (int r = require_ready()) return r;
  if (bytes == 0) return TH_OK;
  TH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx().stream));
  return TH_OK;
}

int th_build_copy(void* dst, const void* src, uint64_t bytes, th_launch** out) {
  *out = nullptr;
  TH_REQUIRE(bytes < (uint64_t(1) << 48), "th_build_copy: too many bytes");
  Builder b("copy", 2);
  CopyArgs a{static_cast<unsigned char*>(dst), static_cast<const unsigned char*>(src), bytes};
  const uint64_t words = (bytes + 15) / 16;
  const unsigned blocks = (unsigned)std::max<uint64_t>(1, std::min<uint64_t>((words + 255) / 256, 4096));
  int k = b.kernel((const void*)th_copy_kernel, "th_copy_kernel", dim3(blocks), dim3(256), 0, a);
  b.ref(0, k, TH_OFFSET(CopyArgs, dst));
  b.ref(1, k, TH_OFFSET(CopyArgs, src));
  b.align(0, 1);
  b.align(1, 1);
  b.work(2.0 * (double)bytes, 0.0, blocks);
  *out = b.release();
  return TH_OK;
}

}  // extern "C"

struct th_arena {
  void* base = nullptr;
  uint64_t bytes = 0;
  std::vector<uint64_t> offsets;
};

// A reserved range of device addresses, mapped to memory as blocks are taken
// from it: every block the pool hands out lies in [base, base + reserved).
struct th_pool {
  int device = 0;
  bool vmm = true;           // a reservation mapped on demand; else one allocation
  void* base = nullptr;
  uint64_t reserved = 0;     // bytes of address space
  uint64_t mapped = 0;       // bytes mapped from base
  uint64_t granularity = 0;
  uint64_t top = 0;          // the end of the highest block taken
  std::vector<std::pair<hipMemGenericAllocationHandle_t, uint64_t>> chunks;
  std::map<uint64_t, uint64_t> free, used;  // offset -> bytes
  // Destroyed while blocks were still taken: the range is released when the
  // last of them is freed (a host's collector may free a pool before its
  // blocks).  Hosts may free from finalizer threads, hence the lock.
  bool closing = false;
  std::mutex mu;
};

// Unmap and free the pool's range, and the pool: once nothing is taken from it.
static int pool_release(th_pool* p) {
  // Nothing may still read the pool's memory.
  TH_HIP(hipDeviceSynchronize());
  if (p->vmm) {
    uint64_t off = 0;
    for (const auto& c : p->chunks) {
      TH_HIP(hipMemUnmap(static_cast<char*>(p->base) + off, c.second));
      TH_HIP(hipMemRelease(c.first));
      off += c.second;
    }
    if (p->base) TH_HIP(hipMemAddressFree(p->base, p->reserved));
  } else if (p->base) {
    TH_HIP(hipFree(p->base));
  }
  delete p;
  return TH_OK;
}

extern "C" {

int th_arena_create(const uint64_t* sizes, int n, uint64_t align, th_arena** out) {
  if (int r = require_ready()) return r;
  *out = nullptr;
  TH_REQUIRE(n >= 0, "th_arena_create: negative slot count");
  if (align < 256) align = 256;
  TH_REQUIRE((align & (align - 1)) == 0, "th_arena_create: alignment must be a power of two");
  th_arena* a = new th_arena();
  uint64_t at = 0;
  for (int i = 0; i < n; ++i) {
    at = (at + align - 1) & ~(align - 1);
    a->offsets.push_back(at);
    at += sizes[i];
  }
  a->bytes = (at + align - 1) & ~(align - 1);
  if (int r = device_alloc(a->bytes, &a->base)) {
    delete a;
    return r;
  }
  *out = a;
  return TH_OK;
}

int th_arena_slot(th_arena* a, int slot, void** out) {
  TH_REQUIRE(a != nullptr, "th_arena_slot: null arena");
  TH_REQUIRE(slot >= 0 && slot < (int)a->offsets.size(), "th_arena_slot: no such slot");
  *out = static_cast<char*>(a->base) + a->offsets[slot];
  return TH_OK;
}

int th_arena_bytes(th_arena* a, uint64_t* out) {
  TH_REQUIRE(a != nullptr, "th_arena_bytes: null arena");
  *out = a->bytes;
  return TH_OK;
}

int th_arena_destroy(th_arena* a) {
  if (!a) return TH_OK;
  if (a->base) TH_HIP(hipFree(a->base));
  delete a;
  return TH_OK;
}

// ---- the slot pool: one reserved range of addresses ---------------------------

int th_pool_create(uint64_t reserve, th_pool** out) {
  if (int r = require_ready()) return r;
  *out = nullptr;
  TH_REQUIRE(reserve > 0, "th_pool_create: reserve some bytes");
  th_pool* p = new th_pool();
  p->device = ctx().device;
  hipMemAllocationProp prop{};
  prop.type = hipMemAllocationTypePinned;
  prop.location.type = hipMemLocationTypeDevice;
  prop.location.id = p->device;
  size_t gran = 0;
  hipError_t e = hipMemGetAllocationGranularity(&gran, &prop, hipMemAllocationGranularityRecommended);
  if (e == hipSuccess && gran > 0) {
    p->granularity = gran;
    p->reserved = (reserve + gran - 1) / gran * gran;
    e = hipMemAddressReserve(&p->base, p->reserved, gran, nullptr, 0);
  }
  if (e != hipSuccess) {
    // No virtual memory management: the whole range as one allocation.
    (void)hipGetLastError();
    p->vmm = false;
    p->reserved = (reserve + 255) / 256 * 256;
    p->granularity = 256;
    if (int r = device_alloc(p->reserved, &p->base)) {
      delete p;
      return r;
    }
    p->mapped = p->reserved;
  }
  *out = p;
  return TH_OK;
}

// Map physical memory behind the reservation up to `end` bytes.
static int pool_map(th_pool* p, uint64_t end) {
  if (end <= p->mapped) return TH_OK;
  if (!p->vmm || end > p->reserved)
    return fail(TH_E_MEMORY, "th_pool_alloc: the pool's " + std::to_string(p->reserved) + " reserved bytes are full");
  uint64_t bytes = std::max<uint64_t>(end - p->mapped, uint64_t(64) << 20);
  bytes = std::min<uint64_t>((bytes + p->granularity - 1) / p->granularity * p->granularity, p->reserved - p->mapped);
  hipMemAllocationProp prop{};
  prop.type = hipMemAllocationTypePinned;
  prop.location.type = hipMemLocationTypeDevice;
  prop.location.id = p->device;
  hipMemGenericAllocationHandle_t h;
  hipError_t e = hipMemCreate(&h, bytes, &prop, 0);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(TH_E_MEMORY, std::string("th_pool_alloc: hipMemCreate of ") + std::to_string(bytes) +
                                 " bytes failed: " + hipGetErrorString(e));
  }
  char* at = static_cast<char*>(p->base) + p->mapped;
  e = hipMemMap(at, bytes, 0, h, 0);
  if (e == hipSuccess) {
    hipMemAccessDesc access{};
    access.location.type = hipMemLocationTypeDevice;
    access.location.id = p->device;
    access.flags = hipMemAccessFlagsProtReadWrite;
    e = hipMemSetAccess(at, bytes, &access, 1);
    if (e != hipSuccess) (void)hipMemUnmap(at, bytes);
  }
  if (e != hipSuccess) {
    (void)hipMemRelease(h);
    return hip_fail(e, "th_pool_alloc: mapping the pool");
  }
  p->chunks.push_back({h, bytes});
  p->mapped += bytes;
  return TH_OK;
}

int th_pool_alloc(th_pool* p, uint64_t bytes, uint64_t align, void** out) {
  if (int r = require_ready()) return r;
  TH_REQUIRE(p != nullptr, "th_pool_alloc: null pool");
  *out = nullptr;
  std::lock_guard<std::mutex> hold(p->mu);
  TH_REQUIRE(!p->closing, "th_pool_alloc: the pool was destroyed");
  if (align < 256) align = 256;
  TH_REQUIRE((align & (align - 1)) == 0, "th_pool_alloc: alignment must be a power of two");
  bytes = std::max<uint64_t>((bytes + 255) / 256 * 256, 256);
  // The first free block that holds it, else past the highest block.
  uint64_t at = UINT64_MAX;
  for (auto it = p->free.begin(); it != p->free.end(); ++it) {
    const uint64_t start = (it->first + align - 1) & ~(align - 1);
    if (start + bytes <= it->first + it->second) {
      at = start;
      const uint64_t lo = it->first, hi = it->first + it->second;
      p->free.erase(it);
      if (start > lo) p->free[lo] = start - lo;
      if (start + bytes < hi) p->free[start + bytes] = hi - (start + bytes);
      break;
    }
  }
  if (at == UINT64_MAX) {
    at = (p->top + align - 1) & ~(align - 1);
    if (int r = pool_map(p, at + bytes)) return r;
    if (at > p->top) p->free[p->top] = at - p->top;
    p->top = at + bytes;
  }
  p->used[at] = bytes;
  *out = static_cast<char*>(p->base) + at;
  return TH_OK;
}

int th_pool_free(th_pool* p, void* ptr) {
  TH_REQUIRE(p != nullptr, "th_pool_free: null pool");
  if (!ptr) return TH_OK;
  bool last = false;
  {
    std::lock_guard<std::mutex> hold(p->mu);
    const uint64_t at = static_cast<uint64_t>(static_cast<char*>(ptr) - static_cast<char*>(p->base));
    auto it = p->used.find(at);
    TH_REQUIRE(ptr >= p->base && it != p->used.end(), "th_pool_free: not a block of this pool");
    uint64_t lo = at, hi = at + it->second;
    p->used.erase(it);
    // Coalesce with the free neighbours; a free block at the top lowers it.
    auto next = p->free.find(hi);
    if (next != p->free.end()) hi += next->second, p->free.erase(next);
    auto prev = p->free.lower_bound(lo);
    if (prev != p->free.begin()) {
      --prev;
      if (prev->first + prev->second == lo) lo = prev->first, p->free.erase(prev);
    }
    if (hi == p->top) p->top = lo;
    else p->free[lo] = hi - lo;
    last = p->closing && p->used.empty();
  }
  return last ? pool_release(p) : TH_OK;
}

int th_pool_info(th_pool* p, void** base, uint64_t* reserved, uint64_t* mapped) {
  TH_REQUIRE(p != nullptr, "th_pool_info: null pool");
  *base = p->base;
  *reserved = p->reserved;
  *mapped = p->mapped;
  return TH_OK;
}

int th_pool_destroy(th_pool* p) {
  if (!p) return TH_OK;
  {
    std::lock_guard<std::mutex> hold(p->mu);
    if (p->closing) return TH_OK;
    p->closing = true;
    // Blocks still taken keep the range: the last th_pool_free releases it.
    if (!p->used.empty()) return TH_OK;
  }
  return pool_release(p);
}

// ---- launches --------------------------------------------------------------

int th_launch_run(th_launch* l) {
  if (int r = require_ready()) return r;
  TH_REQUIRE(l != nullptr, "th_launch_run: null launch");
  if (int r = ensure_workspace(l)) return r;
  for (const Kernel& k : l->kernels)
    if (int r = launch_kernel(k, ctx().stream)) return r;
  return TH_OK;
}

int th_launch_repoint(th_launch* l, int value, void* ptr) {
  TH_REQUIRE(l != nullptr, "th_launch_repoint: null launch");
  TH_REQUIRE(value >= 0 && value < (int)l->values.size(),
             "th_launch_repoint: " + l->name + " has no value " + std::to_string(value));
  TH_REQUIRE(reinterpret_cast<uintptr_t>(ptr) % l->align[value] == 0,
             "th_launch_repoint: " + l->name + " was built for value " + std::to_string(value) +
                 " aligned to " + std::to_string(l->align[value]) + " bytes");
  for (const Ref& r : l->values[value])
    std::memcpy(l->kernels[r.kernel].args + r.offset, &ptr, sizeof(void*));
  return TH_OK;
}

int th_launch_work(th_launch* l, th_work* out) {
  TH_REQUIRE(l != nullptr, "th_launch_work: null launch");
  *out = l->work;
  return TH_OK;
}

int th_launch_describe(th_launch* l, char* out, size_t capacity) {
  TH_REQUIRE(l != nullptr, "th_launch_describe: null launch");
  std::string s = l->name + ":";
  for (const Kernel& k : l->kernels) {
    char buf[160];
    std::snprintf(buf, sizeof buf, " %s<<<(%u,%u,%u),(%u,%u,%u),%u>>>", k.name, k.grid.x, k.grid.y,
                  k.grid.z, k.block.x, k.block.y, k.block.z, k.shmem);
    s += buf;
  }
  std::snprintf(out, capacity, "%s", s.c_str());
  return TH_OK;
}

int th_launch_workspace(th_launch* l, uint64_t* bytes) {
  TH_REQUIRE(l != nullptr && bytes != nullptr, "th_launch_workspace: null argument");
  *bytes = l->ws_bytes;
  return TH_OK;
}

int th_launch_set_workspace(th_launch* l, void* ptr) {
  TH_REQUIRE(l != nullptr, "th_launch_set_workspace: null launch");
  TH_REQUIRE(l->ws_bytes > 0, "th_launch_set_workspace: " + l->name + " has no workspace");
  TH_REQUIRE(ptr != nullptr && reinterpret_cast<uintptr_t>(ptr) % 256 == 0,
             "th_launch_set_workspace: the workspace must be a 256-byte aligned device address");
  if (l->ws_owned) {
    TH_HIP(hipStreamSynchronize(ctx().stream));  // no kernel of this launch still reads the old one
    TH_HIP(hipFree(l->ws));
  }
  l->ws = ptr;
  l->ws_owned = false;
  th::point_workspace(l);
  return TH_OK;
}

int th_launch_destroy(th_launch* l) {
  if (!l) return TH_OK;
  for (void* p : l->owned)
    if (p) TH_HIP(hipFree(p));
  if (l->ws_owned && l->ws) TH_HIP(hipFree(l->ws));
  delete l;
  return TH_OK;
}

}  // extern "C"

// ---- graphs ----------------------------------------------------------------

struct th_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  std::vector<th_launch*> steps;
  std::vector<std::vector<hipGraphNode_t>> nodes;  // per step, per kernel
};

namespace th {

static hipKernelNodeParams node_params(const Kernel& k, void** params) {
  hipKernelNodeParams p{};
  // A module function stands where a kernel's host stub would: the graph
  // resolves it as the function itself.
  p.func = k.module ? static_cast<void*>(k.module) : const_cast<void*>(k.fn);
  p.gridDim = k.grid;
  p.blockDim = k.block;
  p.sharedMemBytes = k.shmem;
  p.kernelParams = params;
  p.extra = nullptr;
  return p;
}

}  // namespace th

extern "C" {

int th_graph_capture(th_launch* const* steps, int n, th_graph** out) {
  if (int r = require_ready()) return r;
  *out = nullptr;
  TH_REQUIRE(n >= 0, "th_graph_capture: negative step count");
  th_graph* g = new th_graph();
  hipError_t e = hipGraphCreate(&g->graph, 0);
  if (e != hipSuccess) {
    delete g;
    return hip_fail(e, "hipGraphCreate");
  }
  hipGraphNode_t last = nullptr;
  for (int i = 0; i < n; ++i) {
    th_launch* l = steps[i];
    if (int r = ensure_workspace(l)) {
      (void)hipGraphDestroy(g->graph);
      delete g;
      return r;
    }
    g->steps.push_back(l);
    g->nodes.emplace_back();
    for (Kernel& k : l->kernels) {
      void* params[1] = {k.args};
      hipKernelNodeParams p = node_params(k, params);
      hipGraphNode_t node;
      e = hipGraphAddKernelNode(&node, g->graph, last ? &last : nullptr, last ? 1 : 0, &p);
      if (e != hipSuccess) {
        (void)hipGraphDestroy(g->graph);
        delete g;
        return hip_fail(e, "hipGraphAddKernelNode");
      }
      g->nodes.back().push_back(node);
      last = node;
    }
  }
  e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g->graph);
    delete g;
    return hip_fail(e, "hipGraphInstantiate");
  }
  // The graph's work descriptions to the device now rather than at the first
  // replay.  (A replay's fixed cost is the host's hipGraphLaunch call, about
  // 15 us for one node plus ~1 us a node here; uploading does not change it.)
  e = hipGraphUpload(g->exec, ctx().stream);
  if (e != hipSuccess) {
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(g->graph);
    delete g;
    return hip_fail(e, "hipGraphUpload");
  }
  *out = g;
  return TH_OK;
}

int th_graph_replay(th_graph* g) {
  if (int r = require_ready()) return r;
  TH_REQUIRE(g != nullptr, "th_graph_replay: null graph");
  TH_HIP(hipGraphLaunch(g->exec, ctx().stream));
  return TH_OK;
}

int th_graph_retarget(th_graph* g, int step) {
  if (int r = require_ready()) return r;
  TH_REQUIRE(g != nullptr, "th_graph_retarget: null graph");
  TH_REQUIRE(step >= 0 && step < (int)g->steps.size(), "th_graph_retarget: no such step");
  th_launch* l = g->steps[step];
  for (size_t j = 0; j < l->kernels.size(); ++j) {
    Kernel& k = l->kernels[j];
    void* params[1] = {k.args};
    hipKernelNodeParams p = node_params(k, params);
    TH_HIP(hipGraphExecKernelNodeSetParams(g->exec, g->nodes[step][j], &p));
  }
  return TH_OK;
}

int th_graph_release(th_graph* g) {
  if (!g) return TH_OK;
  if (g->exec) TH_HIP(hipGraphExecDestroy(g->exec));
  if (g->graph) TH_HIP(hipGraphDestroy(g->graph));
  delete g;
  return TH_OK;
}

}  // extern "C"

// ---- timing ----------------------------------------------------------------

namespace th {

static int ensure_clearing() {
  Context& c = ctx();
  if (c.clear_buf) return TH_OK;
  double cache = (double)c.prop.l2CacheSize + 256.0 * 1024 * 1024;
  size_t bytes = (size_t)(2.0 * cache);
  bytes = (bytes + 4095) & ~(size_t)4095;
  if (int r = device_alloc(bytes, &c.clear_buf)) return r;
  TH_HIP(hipMemsetAsync(c.clear_buf, 0, bytes, c.stream));
  if (int r = device_alloc(sizeof(uint32_t), (void**)&c.sink)) return r;
  c.clear_bytes = bytes;
  return TH_OK;
}

static int clear_cache() {
  Context& c = ctx();
  ClearArgs a{static_cast<const u32x4*>(c.clear_buf), c.sink, c.clear_bytes / 16, 1};
  int blocks = c.prop.multiProcessorCount * 8;
  hipLaunchKernelGGL(th_clear_kernel, dim3(blocks), dim3(256), 0, c.stream, a);
  TH_HIP(hipGetLastError());
  return TH_OK;
}

// Bytes a second read from what the caches hold: 64 MiB (within L2 + MALL)
// read 16 times over in one launch of the clearing kernel, the best of 5
// launches after one, once per process.  The reference takes twice the
// memory's rate for it (ext/CUDAExt.jl:908-921); this is the device's own.
// Timing events, destroyed with the scope, so that every early return
// (TH_HIP's included) releases them; an event still pending on the stream
// is released by HIP once it completes.
struct Events {
  std::vector<hipEvent_t> e;
  explicit Events(size_t n) : e(n, nullptr) {}
  hipError_t create() {
    for (auto& x : e) {
      const hipError_t r = hipEventCreate(&x);
      if (r != hipSuccess) {
        x = nullptr;
        return r;
      }
    }
    return hipSuccess;
  }
  ~Events() {
    for (hipEvent_t x : e)
      if (x) (void)hipEventDestroy(x);
  }
  hipEvent_t operator[](size_t i) const { return e[i]; }
  Events(const Events&) = delete;
  Events& operator=(const Events&) = delete;
};

static int cached_rate(double* out) {
  Context& c = ctx();
  if (c.cached_rate < 0) {
    const uint64_t bytes = std::min<uint64_t>(64ull << 20, c.clear_bytes);
    const int passes = 16;
    ClearArgs a{static_cast<const u32x4*>(c.clear_buf), c.sink, bytes / 16, passes};
    int blocks = c.prop.multiProcessorCount * 8;
    hipLaunchKernelGGL(th_clear_kernel, dim3(blocks), dim3(256), 0, c.stream, a);
    TH_HIP(hipGetLastError());
    Events ev(6);
    TH_HIP(ev.create());
    TH_HIP(hipEventRecord(ev[0], c.stream));
    for (int i = 0; i < 5; ++i) {
      hipLaunchKernelGGL(th_clear_kernel, dim3(blocks), dim3(256), 0, c.stream, a);
      TH_HIP(hipGetLastError());
      TH_HIP(hipEventRecord(ev[i + 1], c.stream));
    }
    TH_HIP(hipEventSynchronize(ev[5]));
    float best = 1e30f;
    for (int i = 0; i < 5; ++i) {
      float ms = 0;
      TH_HIP(hipEventElapsedTime(&ms, ev[i], ev[i + 1]));
      best = std::min(best, ms);
    }
    c.cached_rate = (double)passes * bytes / (best * 1e-3);
  }
  *out = c.cached_rate;
  return TH_OK;
}

// Minimum over `samples` of one replay of `g` after the caches are cleared
// (cleared, ext/CUDAExt.jl:821-833).
static int cleared(th_graph* g, int samples, double* out) {
  Context& c = ctx();
  Events ev(2 * samples);
  TH_HIP(ev.create());
  for (int i = 0; i < samples; ++i) {
    if (int r = clear_cache()) return r;
    TH_HIP(hipEventRecord(ev[2 * i], c.stream));
    TH_HIP(hipGraphLaunch(g->exec, c.stream));
    TH_HIP(hipEventRecord(ev[2 * i + 1], c.stream));
  }
  TH_HIP(hipEventSynchronize(ev[2 * samples - 1]));
  float best = 1e30f;
  for (int i = 0; i < samples; ++i) {
    float ms = 0;
    TH_HIP(hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]));
    best = std::min(best, ms);
  }
  *out = best * 1e-3;
  return TH_OK;
}

static int mean_replay(th_graph* g, int warmup, int reps, double* out) {
  Context& c = ctx();
  for (int i = 0; i < warmup; ++i) TH_HIP(hipGraphLaunch(g->exec, c.stream));
  Events ab(2);
  TH_HIP(ab.create());
  const hipEvent_t a = ab[0], b = ab[1];
  TH_HIP(hipEventRecord(a, c.stream));
  for (int i = 0; i < reps; ++i) TH_HIP(hipGraphLaunch(g->exec, c.stream));
  TH_HIP(hipEventRecord(b, c.stream));
  TH_HIP(hipEventSynchronize(b));
  float ms = 0;
  TH_HIP(hipEventElapsedTime(&ms, a, b));
  *out = ms * 1e-3 / std::max(reps, 1);
  return TH_OK;
}

// What replaying one graph alone adds: an empty kernel's graph timed alone,
// less its time among a long graph of them (replay_overhead,
// ext/CUDAExt.jl:874-884).
static int replay_overhead(double* out) {
  Context& c = ctx();
  if (c.replay_overhead >= 0) {
    *out = c.replay_overhead;
    return TH_OK;
  }
  th_launch blank;
  blank.name = "blank";
  Kernel k;
  k.fn = (const void*)th_blank_kernel;
  k.name = "th_blank_kernel";
  int zero = 0;
  std::memcpy(k.args, &zero, sizeof zero);
  k.args_size = sizeof zero;
  blank.kernels.push_back(k);
  th_launch* one[1] = {&blank};
  th_graph* alone = nullptr;
  if (int r = th_graph_capture(one, 1, &alone)) return r;
  double t_alone = 0;
  int r = cleared(alone, 20, &t_alone);
  th_graph_release(alone);
  if (r) return r;
  std::vector<th_launch*> many(200, &blank);
  th_graph* batch = nullptr;
  if ((r = th_graph_capture(many.data(), (int)many.size(), &batch))) return r;
  double t_batch = 0;
  r = mean_replay(batch, 2, 5, &t_batch);
  th_graph_release(batch);
  if (r) return r;
  c.replay_overhead = std::max(0.0, t_alone - t_batch / many.size());
  // An empty kernel's share of a long graph: the gap between launches inside
  // a replayed graph, the cover's per-launch price (ext/CUDAExt.jl:904-906).
  c.launch_gap = t_batch / many.size();
  // What a replay costs beyond its launches, back to back (a one-launch
  // graph replayed 100 times), and what a direct launch costs back to back:
  // the two sides of graph-or-direct for a recording of K launches.
  if ((r = th_graph_capture(one, 1, &alone))) return r;
  double t_one = 0;
  r = mean_replay(alone, 5, 100, &t_one);
  th_graph_release(alone);
  if (r) return r;
  c.graph_base = std::max(0.0, t_one - c.launch_gap);
  for (int i = 0; i < 5; ++i)
    if ((r = launch_kernel(blank.kernels[0], c.stream))) return r;
  Events ab(2);
  TH_HIP(ab.create());
  const hipEvent_t a = ab[0], b = ab[1];
  TH_HIP(hipEventRecord(a, c.stream));
  for (int i = 0; i < 200; ++i)
    if ((r = launch_kernel(blank.kernels[0], c.stream))) return r;
  TH_HIP(hipEventRecord(b, c.stream));
  TH_HIP(hipEventSynchronize(b));
  float ms = 0;
  TH_HIP(hipEventElapsedTime(&ms, a, b));
  c.direct_gap = ms * 1e-3 / 200;
  *out = c.replay_overhead;
  return TH_OK;
}

}  // namespace th

extern "C" {

int th_time_launch(th_launch* l, int samples, double* seconds) {
  if (int r = require_ready()) return r;
  TH_REQUIRE(l != nullptr, "th_time_launch: null launch");
  std::lock_guard<std::mutex> lock(g_timing);
  Context& c = ctx();
  TH_HIP(hipStreamSynchronize(c.stream));
  if (int r = ensure_clearing()) return r;
  double overhead = 0;
  if (int r = replay_overhead(&overhead)) return r;
  th_launch* one[1] = {l};
  th_graph* g = nullptr;
  if (int r = th_graph_capture(one, 1, &g)) return r;
  if (samples <= 0) {
    // As many samples as fit 10 ms of the launch, 3 to 20.
    double once = 0;
    int r = mean_replay(g, 1, 1, &once);
    if (r) {
      th_graph_release(g);
      return r;
    }
    samples = (int)std::min(20.0, std::max(3.0, 1.0e-2 / std::max(once, 1.0e-6)));
  }
  double t = 0;
  int r = cleared(g, samples, &t);
  th_graph_release(g);
  if (r) return r;
  *seconds = std::max(0.0, t - overhead);
  return TH_OK;
}

int th_dispatch_costs(double* graph_base, double* in_graph, double* direct) {
  if (int r = require_ready()) return r;
  TH_REQUIRE(graph_base && in_graph && direct, "th_dispatch_costs: null output");
  std::lock_guard<std::mutex> lock(g_timing);
  Context& c = ctx();
  TH_HIP(hipStreamSynchronize(c.stream));
  if (int r = ensure_clearing()) return r;
  double overhead = 0;
  if (int r = replay_overhead(&overhead)) return r;
  *graph_base = c.graph_base;
  *in_graph = c.launch_gap;
  *direct = c.direct_gap;
  return TH_OK;
}

int th_matrix_rate(int vary, double* flops_per_s, double* clock_hz) {
  if (int r = require_ready()) return r;
  TH_REQUIRE(flops_per_s && clock_hz, "th_matrix_rate: null output");
  std::lock_guard<std::mutex> lock(g_timing);
  Context& c = ctx();
  const int blocks = 2 * c.prop.multiProcessorCount;
  // Random operand bits: bf16 in [1, 2) with random signs and mantissas.
  std::vector<uint32_t> host(16 * 64 * 4);
  uint64_t z = 0x9e3779b97f4a7c15ull;
  for (uint32_t& w : host) {
    z = z * 6364136223846793005ull + 1442695040888963407ull;
    const uint32_t r = (uint32_t)(z >> 32);
    w = (0x3f803f80u) | (r & 0x807f807fu);
  }
  void* seed = nullptr;
  void* sink = nullptr;
  void* stamps = nullptr;
  if (int r = device_alloc(host.size() * 4, &seed)) return r;
  int rc = device_alloc(blocks * sizeof(float), &sink);
  if (!rc) rc = device_alloc(blocks * 4 * sizeof(uint64_t), &stamps);
  if (rc) {
    (void)hipFree(seed);
    if (sink) (void)hipFree(sink);
    return rc;
  }
  auto done = [&](int r) {
    (void)hipStreamSynchronize(c.stream);
    (void)hipFree(seed);
    (void)hipFree(sink);
    (void)hipFree(stamps);
    return r;
  };
  if (hipMemcpy(seed, host.data(), host.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
    return done(fail(TH_E_STATE, "th_matrix_rate: seed upload failed"));
  const int iters = 20000;
  RateArgs a{static_cast<const u32x4*>(seed), static_cast<float*>(sink), static_cast<uint64_t*>(stamps), iters,
             vary ? 1 : 0};
  Events ev(2);
  if (ev.create() != hipSuccess) return done(fail(TH_E_STATE, "th_matrix_rate: events"));
  hipLaunchKernelGGL(th_matrix_rate_kernel, dim3(blocks), dim3(256), 0, c.stream, a);  // warm up the clocks
  (void)hipEventRecord(ev[0], c.stream);
  hipLaunchKernelGGL(th_matrix_rate_kernel, dim3(blocks), dim3(256), 0, c.stream, a);
  (void)hipEventRecord(ev[1], c.stream);
  if (hipEventSynchronize(ev[1]) != hipSuccess) return done(fail(TH_E_STATE, "th_matrix_rate: run failed"));
  float ms = 0;
  (void)hipEventElapsedTime(&ms, ev[0], ev[1]);
  std::vector<uint64_t> st(blocks * 4);
  if (hipMemcpy(st.data(), stamps, st.size() * 8, hipMemcpyDeviceToHost) != hipSuccess)
    return done(fail(TH_E_STATE, "th_matrix_rate: stamps"));
  double clock = 0;
  for (int i = 0; i < blocks; ++i) clock += (double)(st[4 * i + 1] - st[4 * i]) / (double)(st[4 * i + 3] - st[4 * i + 2]);
  *clock_hz = clock / blocks * 100e6;  // the real-time counter runs at 100 MHz
  *flops_per_s = (double)blocks * 4 * iters * 32 * 32768.0 / (ms * 1e-3);
  return done(TH_OK);
}

int th_lds_rate(int mode, int per_cu, double* bytes_per_s, double* flops_per_s, double* clock_hz) {
  if (int r = require_ready()) return r;
  TH_REQUIRE(bytes_per_s && flops_per_s && clock_hz, "th_lds_rate: null output");
  TH_REQUIRE(mode >= 0 && mode <= 3, "th_lds_rate: mode must be 0 (b128), 1 (tr), 2 (b128 + products) or 3 (tr + products)");
  TH_REQUIRE(per_cu == 1 || per_cu == 2, "th_lds_rate: one or two workgroups a CU");
  std::lock_guard<std::mutex> lock(g_timing);
  Context& c = ctx();
  const int blocks = per_cu * c.prop.multiProcessorCount;
  void* sink = nullptr;
  void* stamps = nullptr;
  if (int r = device_alloc(blocks * sizeof(uint32_t), &sink)) return r;
  if (int r = device_alloc(blocks * 4 * sizeof(uint64_t), &stamps)) {
    (void)hipFree(sink);
    return r;
  }
  auto done = [&](int r) {
    (void)hipStreamSynchronize(c.stream);
    (void)hipFree(sink);
    (void)hipFree(stamps);
    return r;
  };
  const int iters = 4000;
  LdsRateArgs a{static_cast<uint32_t*>(sink), static_cast<uint64_t*>(stamps), iters};
  const void* k = mode == 0 ? (const void*)th_lds_rate_kernel<0>
                : mode == 1 ? (const void*)th_lds_rate_kernel<1>
                : mode == 2 ? (const void*)th_lds_rate_kernel<2>
                            : (const void*)th_lds_rate_kernel<3>;
  void* params[] = {&a};
  Events ev(2);
  if (ev.create() != hipSuccess) return done(fail(TH_E_STATE, "th_lds_rate: events"));
  // Warm up the clocks, then time the second launch.
  if (hipLaunchKernel(k, dim3(blocks), dim3(256), params, 0, c.stream) != hipSuccess)
    return done(fail(TH_E_STATE, "th_lds_rate: launch failed"));
  (void)hipEventRecord(ev[0], c.stream);
  (void)hipLaunchKernel(k, dim3(blocks), dim3(256), params, 0, c.stream);
  (void)hipEventRecord(ev[1], c.stream);
  if (hipEventSynchronize(ev[1]) != hipSuccess) return done(fail(TH_E_STATE, "th_lds_rate: run failed"));
  float ms = 0;
  (void)hipEventElapsedTime(&ms, ev[0], ev[1]);
  std::vector<uint64_t> st(blocks * 4);
  if (hipMemcpy(st.data(), stamps, st.size() * 8, hipMemcpyDeviceToHost) != hipSuccess)
    return done(fail(TH_E_STATE, "th_lds_rate: stamps"));
  double clock = 0;
  for (int i = 0; i < blocks; ++i) clock += (double)(st[4 * i + 1] - st[4 * i]) / (double)(st[4 * i + 3] - st[4 * i + 2]);
  *clock_hz = clock / blocks * 100e6;
  const double reads = (double)blocks * 4 * 8 * iters;  // wave reads of 1 KB
  *bytes_per_s = reads * 1024.0 / (ms * 1e-3);
  *flops_per_s = mode >= 2 ? reads * 32768.0 / (ms * 1e-3) : 0.0;
  return done(TH_OK);
}

int th_read_rate(int mode, double* bytes_per_s) {
  if (int r = require_ready()) return r;
  TH_REQUIRE(bytes_per_s, "th_read_rate: null output");
  TH_REQUIRE(mode == 0 || mode == 1, "th_read_rate: mode must be 0 (a 2 MB stream a wave) or 1 (the dQ sweep's dS' reads)");
  std::lock_guard<std::mutex> lock(g_timing);
  Context& c = ctx();
  const int cus = c.prop.multiProcessorCount;
  // Mode 1's array is B 8 x H 16 x S^2 bf16 (4 GiB); mode 0's one 2 MB stream a wave.
  const size_t bytes = mode == 1 ? (size_t)8 * 16 * 4096 * 4096 * 2 : (size_t)cus * 4 * 2 * 1024 * 1024;
  const size_t lds = 96 * 1024;  // one workgroup a CU
  TH_HIP(hipFuncSetAttribute((const void*)th_read_rate_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  void* src = nullptr;
  void* sink = nullptr;
  if (int r = device_alloc(bytes, &src)) return r;
  if (int r = device_alloc(4096 * sizeof(uint32_t), &sink)) {
    (void)hipFree(src);
    return r;
  }
  auto done = [&](int r) {
    (void)hipStreamSynchronize(c.stream);
    (void)hipFree(src);
    (void)hipFree(sink);
    return r;
  };
  ReadRateArgs a{static_cast<const u32x4*>(src), static_cast<uint32_t*>(sink), mode};
  const dim3 grid = mode == 1 ? dim3(8, 16, 8) : dim3(cus);
  // Bytes read: mode 0 the whole array; mode 1, per (batch, head), four waves
  // of each workgroup x read (4 x + 4) + (4 (15 - x) + 4) steps of 8 KB.
  double read = (double)bytes;
  if (mode == 1) {
    read = 0;
    for (int x = 0; x < 8; ++x) read += 4.0 * ((4 * x + 4) + (4 * (15 - x) + 4)) * 8192;
    read *= 8 * 16;
  }
  void* params[] = {&a};
  Events ev(2);
  if (ev.create() != hipSuccess) return done(fail(TH_E_STATE, "th_read_rate: events"));
  if (hipLaunchKernel((const void*)th_read_rate_kernel, grid, dim3(256), params, lds, c.stream) != hipSuccess)
    return done(fail(TH_E_STATE, "th_read_rate: launch failed"));
  (void)hipEventRecord(ev[0], c.stream);
  for (int r = 0; r < 5; ++r) (void)hipLaunchKernel((const void*)th_read_rate_kernel, grid, dim3(256), params, lds, c.stream);
  (void)hipEventRecord(ev[1], c.stream);
  if (hipEventSynchronize(ev[1]) != hipSuccess) return done(fail(TH_E_STATE, "th_read_rate: run failed"));
  float ms = 0;
  (void)hipEventElapsedTime(&ms, ev[0], ev[1]);
  *bytes_per_s = 5.0 * read / (ms * 1e-3);
  return done(TH_OK);
}

int th_time_graph(th_graph* g, int warmup, int reps, double* seconds) {
  if (int r = require_ready()) return r;
  TH_REQUIRE(g != nullptr, "th_time_graph: null graph");
  TH_REQUIRE(reps > 0 && warmup >= 0, "th_time_graph: reps must be positive");
  std::lock_guard<std::mutex> lock(g_timing);
  return mean_replay(g, warmup, reps, seconds);
}

int th_time_run(th_launch* l, int warmup, int reps, double* seconds) {
  if (int r = require_ready()) return r;
  TH_REQUIRE(l != nullptr, "th_time_run: null launch");
  TH_REQUIRE(reps > 0 && warmup >= 0, "th_time_run: reps must be positive");
  std::lock_guard<std::mutex> lock(g_timing);
  Context& c = ctx();
  for (int i = 0; i < warmup; ++i)
    if (int r = th_launch_run(l)) return r;
  Events ab(2);
  TH_HIP(ab.create());
  const hipEvent_t a = ab[0], b = ab[1];
  TH_HIP(hipEventRecord(a, c.stream));
  for (int i = 0; i < reps; ++i)
    if (int r = th_launch_run(l)) return r;
  TH_HIP(hipEventRecord(b, c.stream));
  TH_HIP(hipEventSynchronize(b));
  float ms = 0;
  TH_HIP(hipEventElapsedTime(&ms, a, b));
  *seconds = ms * 1e-3 / reps;
  return TH_OK;
}

}  // extern "C"
