// Allocation-free decode-shape bf16 GEMM, for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops, harnesses
// that forbid hipMalloc).  The reference has no counterpart.
//
// catena_mi355x_gemm_bf16 (n <= 16) keeps its split-K partials in a
// pool-backed workspace that it grows with hipMalloc on first use; this
// variant keeps them in `scratch`, a fixed array in device memory that every
// GPU the library runs on holds from the time the library's code object is
// loaded until the process ends.  It launches the same kernels, so it gives
// the same bits.
//
// The array's name is only a host-side stand-in for the device symbol: host
// code never passes it to a kernel or a copy.  catena_mi355x_init (through
// noalloc_setup, with the device current) looks up the array's device
// address once per device with hipGetSymbolAddress, and the entry point
// passes that address to the kernels.  Every call on a device shares that
// device's array: calls that overlap on one device race.  With a k split the
// plain-output path writes every workgroup's f32 partial to the array and a
// second launch adds them (ascending k group): no completion counters, and
// the partials need no clearing (every one is written before it is read).
// Shapes whose partials exceed the array are refused before any launch
// (catena_mi355x_gemm_bf16_decode_plan reports the partials' size).
#include <hip/hip_runtime.h>

#include "internal.h"

namespace catena {
namespace {
// Partials of S k groups x n rows x m columns (f32).  The k split spreads
// about 256 workgroups, so most decode shapes stay near 2 MiB at 16 rows,
// but the rounding of the split can exceed 4 MiB (16 x 24224 x 2056 needs
// 4.4 MiB): such shapes are refused.
constexpr uint64_t kScratchBytes = 4ull << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
void* g_scratch_addr[kMaxDevices] = {};
}  // namespace

int noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices)
    return fail(CATENA_ERR_UNSUPPORTED, "device index %d beyond %d", device, kMaxDevices);
  if (g_scratch_addr[device]) return CATENA_OK;
  void* addr = nullptr;
  const int st = hip_check(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)),
                           "hipGetSymbolAddress(scratch)");
  if (st) return st;
  if (!addr) return fail(CATENA_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
  g_scratch_addr[device] = addr;
  return CATENA_OK;
}

void* noalloc_scratch(int device) {
  return device >= 0 && device < kMaxDevices ? g_scratch_addr[device] : nullptr;
}

uint64_t noalloc_scratch_bytes() { return kScratchBytes; }

}  // namespace catena

using namespace catena;

extern "C" {

int catena_mi355x_gemm_bf16_decode_noalloc(const uint16_t* a, const uint16_t* b, void* c,
                                           uint64_t n, uint64_t m, uint64_t k, int out_f32) {
  Device& d = device();
  // no implicit init here: init allocates (stream, counters, modules)
  if (!d.ready.load(std::memory_order_acquire))
    return fail(CATENA_ERR_NOT_INITIALIZED, "call catena_mi355x_init before the allocation-free GEMM");
  if (n == 0 || m == 0) return CATENA_OK;
  if (!a || !b || !c) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  if (n > 16 || k == 0 || m % 8 != 0 || k % 8 != 0)
    return fail(CATENA_ERR_INVALID_ARGUMENT,
                "allocation-free GEMM takes decode shapes only (n <= 16, m %% 8 == 0, k %% 8 == 0, "
                "k > 0)");
  void* s = noalloc_scratch(d.device);
  if (!s) return fail(CATENA_ERR_NOT_INITIALIZED, "scratch address not set up for device %d", d.device);
  // the size limit is checked before any launch, inside gemm_bf16_decode
  return gemm_bf16_decode(a, b, c, n, m, k,
                          out_f32 ? DecodeEpilogue::StoreF32 : DecodeEpilogue::StoreBf16,
                          DecodeEpiArgs{}, s, kScratchBytes);
}

}  // extern "C"
