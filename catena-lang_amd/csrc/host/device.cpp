// Device, module loader, buffer pool and kernel ABI of libcatena_mi355x.
//
// Replaces three reference mechanisms:
//  * per-Runtime hipcc build + dlopen of generated code
//    (catena-lang/src/runtime/artifact.rs:44-103, runtime.rs:249-263): the
//    hand-written gfx950 kernels are compiled once at build time into code
//    objects next to this library and loaded with hipModuleLoad; launches go
//    through hipModuleLaunchKernel on one library-owned stream;
//  * hipMallocManaged per buffer + hipFree on drop
//    (catena-lang/src/runtime/mem.rs:119-125, :152-171): a size-classed
//    device pool with cached free lists, stream-ordered reuse;
//  * raw host dereference of managed memory in to_f32_vec / to_u64_vec
//    (catena-lang/src/runtime/mem.rs:44-70): explicit synchronous copies.
#include "internal.h"

#include <dlfcn.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace catena {

static thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

void clear_error() { g_last_error.clear(); }
const char* last_error() { return g_last_error.c_str(); }

// ------------------------------------------------------------------ device

namespace {
struct KernelSpec {
  KernelId id;
  const char* module;
  const char* symbol;
};

const KernelSpec kKernels[] = {
    {KernelId::GemmF32Exact, "gemm_f32_exact", "catena_gemm_f32_exact"},
    {KernelId::GemmF32ExactT16, "gemm_f32_exact", "catena_gemm_f32_exact_t16"},
    {KernelId::GemmF32ExactQ16, "gemm_f32_exact", "catena_gemm_f32_exact_q16"},
    {KernelId::GemmBf16EdgeBf16, "gemm_bf16", "catena_gemm_bf16_edge_bf16out"},
    {KernelId::GemmBf16EdgeF32, "gemm_bf16", "catena_gemm_bf16_edge_f32out"},
    {KernelId::GemmBf16LdsBf16, "gemm_bf16_lds", "catena_gemm_bf16_lds_bf16out"},
    {KernelId::GemmBf16LdsF32, "gemm_bf16_lds", "catena_gemm_bf16_lds_f32out"},
    {KernelId::GemmBf16K32Bf16, "gemm_bf16_k32", "catena_gemm_bf16_k32_bf16out"},
    {KernelId::GemmBf16K32F32, "gemm_bf16_k32", "catena_gemm_bf16_k32_f32out"},
    {KernelId::GemmBf16K32N128Bf16, "gemm_bf16_k32", "catena_gemm_bf16_k32n128_bf16out"},
    {KernelId::GemmBf16K32N128F32, "gemm_bf16_k32", "catena_gemm_bf16_k32n128_f32out"},
    {KernelId::GemmBf16K32Silu, "gemm_bf16_k32", "catena_gemm_bf16_k32_silu"},
    {KernelId::GemmBf16K32N128Silu, "gemm_bf16_k32", "catena_gemm_bf16_k32n128_silu"},
    {KernelId::GemmBf16K32N128Rope, "gemm_bf16_k32", "catena_gemm_bf16_k32n128_rope"},
    {KernelId::GemmBf16K32F32Parts, "gemm_bf16_k32", "catena_gemm_bf16_k32_f32parts"},
    {KernelId::GemmBf16DecodeF32, "gemm_bf16_decode", "catena_gemm_bf16_decode_f32out"},
    {KernelId::GemmBf16DecodeBf16, "gemm_bf16_decode", "catena_gemm_bf16_decode_bf16out"},
    {KernelId::GemmBf16DecodeRope, "gemm_bf16_decode", "catena_gemm_bf16_decode_rope"},
    {KernelId::GemmBf16DecodeSilu, "gemm_bf16_decode", "catena_gemm_bf16_decode_silu"},
    {KernelId::GemmBf16DecodeArgmax, "gemm_bf16_decode", "catena_gemm_bf16_decode_argmax"},
    {KernelId::GemmBf16DecodeParts, "gemm_bf16_decode", "catena_gemm_bf16_decode_parts"},
    {KernelId::GemmBf16DecodePartsNt, "gemm_bf16_decode", "catena_gemm_bf16_decode_parts_nt"},
    {KernelId::ArgmaxCompose, "gemm_bf16_decode", "catena_argmax_compose"},
    {KernelId::DecodeReduce, "gemm_bf16_decode", "catena_decode_reduce"},
    {KernelId::AttnDecodeD128, "attn_decode", "catena_attn_decode_bf16_d128"},
    {KernelId::AttnFewD128F32, "attn_few", "catena_attn_few_bf16_d128_f32out"},
    {KernelId::AttnFewD128Bf16, "attn_few", "catena_attn_few_bf16_d128_bf16out"},
    {KernelId::AttnFewSplitD128F32, "attn_few", "catena_attn_few_split_bf16_d128_f32out"},
    {KernelId::AttnFewSplitD128Bf16, "attn_few", "catena_attn_few_split_bf16_d128_bf16out"},
    {KernelId::AttnCausalD128F32, "attn_decode", "catena_attn_causal_bf16_d128_f32out"},
    {KernelId::AttnCausalD128Bf16, "attn_decode", "catena_attn_causal_bf16_d128_bf16out"},
    {KernelId::AttnPrefillD128F32, "attn_prefill", "catena_attn_prefill_bf16_d128_f32out"},
    {KernelId::AttnPrefillD128Bf16, "attn_prefill", "catena_attn_prefill_bf16_d128_bf16out"},
    {KernelId::EmbedRowsBf16, "block", "catena_embed_rows_bf16"},
    {KernelId::RmsnormRows, "block", "catena_rmsnorm_rows"},
    {KernelId::RopeQkvStore, "block", "catena_rope_qkv_store"},
    {KernelId::RopeTable, "block", "catena_rope_table"},
    {KernelId::SiluMulBf16, "block", "catena_silu_mul_bf16"},
    {KernelId::ArgmaxRowsF32, "block", "catena_argmax_rows_f32"},
    {KernelId::BroadcastF32, "tensor", "catena_broadcast_f32"},
    {KernelId::ArangeF32, "tensor", "catena_arange_f32"},
    {KernelId::CopyF32, "tensor", "catena_copy_f32"},
    {KernelId::SumRowsF32, "tensor", "catena_sum_rows_f32"},
    {KernelId::MaxRowsF32, "tensor", "catena_max_rows_f32"},
    {KernelId::SumRowsU64, "tensor", "catena_sum_rows_u64"},
    {KernelId::SoftmaxRows, "softmax", "catena_softmax_rows_f32"},
    {KernelId::ExpApprox, "softmax", "catena_exp_approx_f32"},
    {KernelId::MapF32, "softmax", "catena_map_f32"},
    {KernelId::FillNormalBf16, "fill", "catena_fill_normal_bf16"},
    {KernelId::FillUniformF32, "fill", "catena_fill_uniform_f32"},
    {KernelId::Copy16, "fill", "catena_copy_16b"},
};

std::string library_dir() {
  const char* env = getenv("CATENA_MI355X_KERNEL_DIR");
  if (env && *env) return env;
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&catena_mi355x_init), &info) && info.dli_fname) {
    std::string p = info.dli_fname;
    size_t slash = p.rfind('/');
    if (slash != std::string::npos) return p.substr(0, slash);
  }
  return ".";
}
}  // namespace

Device& device() {
  static Device d;
  return d;
}

int ensure_init() {
  Device& d = device();
  if (d.ready.load(std::memory_order_acquire)) return CATENA_OK;
  return catena_mi355x_init(0);
}

int hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return CATENA_OK;
  return fail(CATENA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int launch(KernelId id, dim3 grid, dim3 block, size_t lds, void** args) {
  Device& d = device();
  hipFunction_t f = d.fn[static_cast<int>(id)];
  if (!f) return fail(CATENA_ERR_LOAD, "kernel %d not loaded", static_cast<int>(id));
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return CATENA_OK;
  hipError_t e = hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                       (unsigned)lds, d.stream, args, nullptr);
  return hip_check(e, "hipModuleLaunchKernel");
}

// ------------------------------------------------------------------ pool

namespace {
struct Pool {
  std::mutex mu;
  std::unordered_map<uint64_t, std::vector<void*>> free_lists;  // class size -> blocks
  std::unordered_map<void*, uint64_t> live;                      // ptr -> class size
  uint64_t bytes_live = 0, bytes_cached = 0, device_allocs = 0;
};
Pool& pool() {
  static Pool p;
  return p;
}

// Size classes: powers of two from 256 B to 64 MiB, then 2 MiB multiples.
uint64_t size_class(uint64_t len) {
  if (len <= 256) return 256;
  if (len <= (64ull << 20)) {
    uint64_t c = 256;
    while (c < len) c <<= 1;
    return c;
  }
  const uint64_t g = 2ull << 20;
  return (len + g - 1) / g * g;
}
}  // namespace

int pool_alloc(uint64_t len, void** out) {
  *out = nullptr;
  if (len == 0) return CATENA_OK;
  int st = ensure_init();
  if (st) return st;
  const uint64_t cls = size_class(len);
  Pool& p = pool();
  {
    std::lock_guard<std::mutex> g(p.mu);
    auto it = p.free_lists.find(cls);
    if (it != p.free_lists.end() && !it->second.empty()) {
      *out = it->second.back();
      it->second.pop_back();
      p.bytes_cached -= cls;
      p.live[*out] = cls;
      p.bytes_live += cls;
      return CATENA_OK;
    }
  }
  void* ptr = nullptr;
  hipError_t e = hipMalloc(&ptr, cls);
  if (e != hipSuccess) {
    // one retry after releasing cached blocks
    catena_pool_trim();
    e = hipMalloc(&ptr, cls);
    if (e != hipSuccess)
      return fail(CATENA_ERR_OUT_OF_MEMORY, "hipMalloc(%llu): %s", (unsigned long long)cls,
                  hipGetErrorString(e));
  }
  std::lock_guard<std::mutex> g(p.mu);
  p.live[ptr] = cls;
  p.bytes_live += cls;
  p.device_allocs += 1;
  *out = ptr;
  return CATENA_OK;
}

int pool_free(void* ptr) {
  if (!ptr) return CATENA_OK;
  Pool& p = pool();
  std::lock_guard<std::mutex> g(p.mu);
  auto it = p.live.find(ptr);
  if (it == p.live.end()) return fail(CATENA_ERR_INVALID_ARGUMENT, "free of a pointer the pool does not own");
  const uint64_t cls = it->second;
  p.live.erase(it);
  p.bytes_live -= cls;
  p.free_lists[cls].push_back(ptr);
  p.bytes_cached += cls;
  return CATENA_OK;
}

uint64_t pool_capacity(void* ptr) {
  Pool& p = pool();
  std::lock_guard<std::mutex> g(p.mu);
  auto it = p.live.find(ptr);
  return it == p.live.end() ? 0 : it->second;
}

// Library-held scratch (split-K partials): grown on demand, never shrunk
// while the library is loaded.  The caller holds Device::ws_mu until it has
// enqueued the launch that uses the block.
int workspace(uint64_t bytes, void** out) {
  Device& d = device();
  if (bytes <= d.ws_bytes) {
    *out = d.ws;
    return CATENA_OK;
  }
  if (d.ws) {
    // queued kernels may still read the old block: wait before releasing it
    int st = hip_check(hipStreamSynchronize(d.stream), "hipStreamSynchronize");
    if (st) return st;
    pool_free(d.ws);
    d.ws = nullptr;
    d.ws_bytes = 0;
  }
  void* p = nullptr;
  int st = pool_alloc(bytes, &p);
  if (st) return st;
  d.ws = p;
  d.ws_bytes = size_class(bytes);
  *out = p;
  return CATENA_OK;
}

}  // namespace catena

using namespace catena;

extern "C" {

namespace {
std::mutex g_init_mu;  // serialises init and shutdown

// Release what init set up (loaded modules, ticket block, stream); used to
// undo a partial init and by shutdown.
void release_device(Device& d) {
  for (int i = 0; i < d.n_modules; ++i) hipModuleUnload(d.modules[i]);
  d.n_modules = 0;
  if (d.small) hipFree(d.small);
  d.small = nullptr;
  if (d.stream) hipStreamDestroy(d.stream);
  d.stream = nullptr;
  for (hipFunction_t& f : d.fn) f = nullptr;
}

int init_failed(int status) {
  release_device(device());
  return status;
}
}  // namespace

int catena_mi355x_init(int device_index) {
  Device& d = device();
  std::lock_guard<std::mutex> g(g_init_mu);
  if (d.ready.load(std::memory_order_acquire)) return CATENA_OK;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
    return fail(CATENA_ERR_NOT_INITIALIZED, "no HIP device visible");
  if (device_index < 0 || device_index >= count)
    return fail(CATENA_ERR_INVALID_ARGUMENT, "device %d out of range (%d devices)", device_index, count);
  int st = hip_check(hipSetDevice(device_index), "hipSetDevice");
  if (st) return st;
  hipDeviceProp_t prop;
  st = hip_check(hipGetDeviceProperties(&prop, device_index), "hipGetDeviceProperties");
  if (st) return st;
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(CATENA_ERR_UNSUPPORTED, "device %d is %s; this library is built for gfx950 only",
                device_index, prop.gcnArchName);
  d.max_lds = prop.sharedMemPerBlock;
  d.cu_count = prop.multiProcessorCount;
  st = hip_check(hipStreamCreateWithFlags(&d.stream, hipStreamNonBlocking), "hipStreamCreate");
  if (st) return init_failed(st);
  void* small = nullptr;
  st = hip_check(hipMalloc(&small, Device::kSmallBytes), "hipMalloc(tickets)");
  if (st) return init_failed(st);
  d.small = static_cast<unsigned char*>(small);
  st = hip_check(hipMemset(small, 0, Device::kSmallBytes), "hipMemset(tickets)");
  if (st) return init_failed(st);
  const std::string dir = library_dir();
  std::unordered_map<std::string, hipModule_t> modules;
  for (const KernelSpec& k : kKernels) {
    auto it = modules.find(k.module);
    if (it == modules.end()) {
      if (d.n_modules == Device::kMaxModules)
        return init_failed(fail(CATENA_ERR_LOAD, "more than %d code objects", Device::kMaxModules));
      const std::string path = dir + "/" + k.module + ".co";
      hipModule_t m = nullptr;
      hipError_t e = hipModuleLoad(&m, path.c_str());
      if (e != hipSuccess)
        return init_failed(fail(CATENA_ERR_LOAD, "hipModuleLoad(%s): %s", path.c_str(),
                                hipGetErrorString(e)));
      d.modules[d.n_modules++] = m;
      it = modules.emplace(k.module, m).first;
    }
    hipFunction_t f = nullptr;
    hipError_t e = hipModuleGetFunction(&f, it->second, k.symbol);
    if (e != hipSuccess)
      return init_failed(fail(CATENA_ERR_LOAD, "hipModuleGetFunction(%s): %s", k.symbol,
                              hipGetErrorString(e)));
    d.fn[static_cast<int>(k.id)] = f;
  }
  // the allocation-free entry point's scratch: its address on this device
  st = noalloc_setup(device_index);
  if (st) return init_failed(st);
  d.device = device_index;
  d.ready.store(true, std::memory_order_release);
  clear_error();
  return CATENA_OK;
}

int catena_mi355x_shutdown(void) {
  Device& d = device();
  std::lock_guard<std::mutex> g(g_init_mu);
  if (!d.ready.load(std::memory_order_acquire)) return CATENA_OK;
  // every queued kernel has finished before anything it may use goes away
  const int st = hip_check(hipStreamSynchronize(d.stream), "hipStreamSynchronize");
  {
    std::lock_guard<std::mutex> ws(d.ws_mu);
    if (d.ws) pool_free(d.ws);
    d.ws = nullptr;
    d.ws_bytes = 0;
  }
  catena_pool_trim();  // cached blocks go back to the device
  d.ready.store(false, std::memory_order_release);
  release_device(d);
  d.device = -1;
  return st;
}

const char* catena_mi355x_last_error(void) { return last_error(); }

void* catena_mi355x_stream(void) {
  if (ensure_init()) return nullptr;
  return device().stream;
}

int catena_mi355x_synchronize(void) {
  int st = ensure_init();
  if (st) return st;
  return hip_check(hipStreamSynchronize(device().stream), "hipStreamSynchronize");
}

int catena_mem_alloc(uint64_t len, catena_mem_t* out) {
  if (!out) return fail(CATENA_ERR_INVALID_ARGUMENT, "out is NULL");
  out->data = nullptr;
  out->len = 0;
  void* p = nullptr;
  int st = pool_alloc(len, &p);
  if (st) return st;
  out->data = p;
  out->len = len;
  return CATENA_OK;
}

int catena_mem_free(catena_mem_t* mem) {
  if (!mem) return CATENA_OK;
  int st = pool_free(mem->data);
  if (st) return st;
  mem->data = nullptr;
  mem->len = 0;
  return CATENA_OK;
}

int catena_mem_write(catena_mem_t mem, uint64_t offset, const void* src, uint64_t len) {
  if (len == 0) return CATENA_OK;
  if (!mem.data || offset > mem.len || len > mem.len - offset || !src)
    return fail(CATENA_ERR_INVALID_ARGUMENT, "write of %llu bytes at %llu outside a %llu-byte buffer",
                (unsigned long long)len, (unsigned long long)offset, (unsigned long long)mem.len);
  int st = ensure_init();
  if (st) return st;
  Device& d = device();
  st = hip_check(hipMemcpyAsync(static_cast<char*>(mem.data) + offset, src, len,
                                hipMemcpyHostToDevice, d.stream),
                 "hipMemcpyAsync(H2D)");
  if (st) return st;
  return hip_check(hipStreamSynchronize(d.stream), "hipStreamSynchronize");
}

int catena_mem_read(catena_mem_t mem, uint64_t offset, void* dst, uint64_t len) {
  if (len == 0) return CATENA_OK;
  if (!mem.data || offset > mem.len || len > mem.len - offset || !dst)
    return fail(CATENA_ERR_INVALID_ARGUMENT, "read of %llu bytes at %llu outside a %llu-byte buffer",
                (unsigned long long)len, (unsigned long long)offset, (unsigned long long)mem.len);
  int st = ensure_init();
  if (st) return st;
  Device& d = device();
  st = hip_check(hipMemcpyAsync(dst, static_cast<const char*>(mem.data) + offset, len,
                                hipMemcpyDeviceToHost, d.stream),
                 "hipMemcpyAsync(D2H)");
  if (st) return st;
  return hip_check(hipStreamSynchronize(d.stream), "hipStreamSynchronize");
}

int catena_pool_stats(uint64_t* bytes_live, uint64_t* bytes_cached, uint64_t* device_allocs) {
  Pool& p = pool();
  std::lock_guard<std::mutex> g(p.mu);
  if (bytes_live) *bytes_live = p.bytes_live;
  if (bytes_cached) *bytes_cached = p.bytes_cached;
  if (device_allocs) *device_allocs = p.device_allocs;
  return CATENA_OK;
}

int catena_pool_trim(void) {
  Device& d = device();
  if (!d.ready.load(std::memory_order_acquire)) return CATENA_OK;
  int st = hip_check(hipStreamSynchronize(d.stream), "hipStreamSynchronize");
  if (st) return st;
  Pool& p = pool();
  std::lock_guard<std::mutex> g(p.mu);
  for (auto& kv : p.free_lists) {
    for (void* ptr : kv.second) {
      hipFree(ptr);
      p.bytes_cached -= kv.first;
    }
    kv.second.clear();
  }
  return CATENA_OK;
}

}  // extern "C"
