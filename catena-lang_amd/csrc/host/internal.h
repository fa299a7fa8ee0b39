// Internal declarations shared by the host-side translation units of
// libcatena_mi355x (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "catena_mi355x.h"

namespace catena {

enum class KernelId : int {
  GemmF32Exact = 0,
  GemmBf16TileBf16,
  GemmBf16TileF32,
  GemmBf16EdgeBf16,
  GemmBf16EdgeF32,
  GemmBf16LdsV0Bf16,  // direct-to-LDS tile kernels, scheduling variants (see kernels.cpp)
  GemmBf16LdsV1Bf16,
  GemmBf16LdsV2Bf16,
  GemmBf16LdsV3Bf16,
  GemmBf16LdsV4Bf16,
  GemmBf16LdsV5Bf16,
  GemmBf16LdsV7Bf16,
  GemmBf16LdsV0F32,
  GemmBf16LdsV1F32,
  GemmBf16LdsV2F32,
  GemmBf16LdsV3F32,
  GemmBf16LdsV4F32,
  GemmBf16LdsV5F32,
  GemmBf16LdsV7F32,
  GemmBf16DeepBf16,
  GemmBf16DeepF32,
  GemmBf16DeepFrontBf16,
  GemmBf16DeepFrontF32,
  GemmBf16Decode,
  GemmBf16DecodeReduce,
  AttnDecodeD128,
  AttnDecodeD128KC,
  AttnCausalD128F32,
  AttnCausalD128Bf16,
  EmbedRowsBf16,
  RmsnormRows,
  RopeQkvStore,
  SiluMulBf16,
  ArgmaxRowsF32,
  SoftmaxRows,
  ExpApprox,
  FillNormalBf16,
  FillUniformF32,
  Copy16,
  Count
};

struct Device {
  bool ready = false;
  int device = -1;
  hipStream_t stream = nullptr;
  size_t max_lds = 0;
  int cu_count = 0;
  hipFunction_t fn[static_cast<int>(KernelId::Count)] = {};
  void* ws = nullptr;  // split-K partials
  uint64_t ws_bytes = 0;
};

Device& device();
int ensure_init();
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
const char* last_error();
int hip_check(hipError_t e, const char* what);
int launch(KernelId id, dim3 grid, dim3 block, size_t lds, void** args);
int pool_alloc(uint64_t len, void** out);
int pool_free(void* ptr);
uint64_t pool_capacity(void* ptr);
int workspace(uint64_t bytes, void** out);

// Fail-stop used by the program ABI: message on stderr, then trap, like
// catena_assert / catena_host_gpu_check (catena-lang/src/codegen/prelude.rs:38-55).
[[noreturn]] void trap_assert(const char* what);
[[noreturn]] void trap_gpu(const char* what);

}  // namespace catena
