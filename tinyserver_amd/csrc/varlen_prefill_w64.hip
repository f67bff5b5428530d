// The 64-rows-per-wave varlen prefill kernel (prefill_w64_body in
// varlen_prefill_w64.h) and its launch.
#include <cstdlib>

#include "tsa_common.h"
#include "varlen_prefill_w64.h"

namespace tsa {

static_assert(kW64MaxSeqs == kW64MaxSeqsHost, "one sequence limit");

// One 4-wave workgroup per CU, one wave per SIMD.
template <typename T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void varlen_prefill_w64(
    PrefillArgs a, const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k) {
  __shared__ __align__(16) char smem[w64_smem_bytes()];
  prefill_w64_body<T>(a, cu_q, cu_k, smem);
}

int prefill_w64_launch(const PrefillArgs& a, bool bf16, hipStream_t stream) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  if (bf16) varlen_prefill_w64<bf16_t><<<dim3(cus), dim3(256), 0, stream>>>(a, a.cu_q, a.cu_k);
  else varlen_prefill_w64<f16_t><<<dim3(cus), dim3(256), 0, stream>>>(a, a.cu_q, a.cu_k);
  return check_launch("tsa_varlen_prefill");
}

// TSA_PREFILL_W64=0 in the environment routes calls to varlen_prefill_gqa
// instead (read once per process).
bool prefill_w64_enabled() {
  static const bool on = [] {
    const char* e = getenv("TSA_PREFILL_W64");
    return !(e && e[0] == '0');
  }();
  return on;
}

}  // namespace tsa
