// pto_ns5_noalloc: NS5 for callers that cannot allocate device memory. It
// has no counterpart in the reference.
//
// The scratch array lives in this translation unit, whose code object holds
// no kernels: the runtime loads a code object onto a GPU when one of its
// symbols is first used there, so the array takes HBM only on GPUs where a
// no-alloc call has looked up its address, not in every process that runs
// the library's NS5 kernels. The kernels themselves come from ns5.hip.
#include <mutex>
#include <string>

#include "pto_common.h"

namespace pto {

// One array per GPU, allocated when this code object is loaded on that GPU
// and held until the process ends; every no-alloc call on a GPU shares it
// (calls that overlap on one GPU race).
constexpr size_t kNs5ScratchBytes = size_t(256) << 20;
static __device__ __align__(256) unsigned char scratch[kNs5ScratchBytes];

namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices];  // device address of `scratch`, per device

// Device address of the scratch on the stream's device, looked up once per
// device with that device current. Host code never uses the array's name as
// an address.
int scratch_ptr(hipStream_t stream, void** ptr) {
  int dev = 0;
  if (stream != nullptr) {
    PTO_HIP(hipStreamGetDevice(stream, &dev));
  } else {
    PTO_HIP(hipGetDevice(&dev));
  }
  PTO_REQUIRE(dev >= 0 && dev < kScratchDevices, "newton_schulz_orthogonalize (no-alloc): device ordinal out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int prev = 0;
    PTO_HIP(hipGetDevice(&prev));
    if (prev != dev) PTO_HIP(hipSetDevice(dev));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (prev != dev) PTO_HIP(hipSetDevice(prev));
    PTO_HIP(e);
    PTO_REQUIRE(p != nullptr && (reinterpret_cast<uintptr_t>(p) & 255) == 0,
                "newton_schulz_orthogonalize (no-alloc): scratch address not 256-byte aligned");
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return 0;
}

}  // namespace
}  // namespace pto

extern "C" int pto_ns5_noalloc(const void* G, void* out, int dtype, int64_t batch, int64_t rows, int64_t cols,
                               int64_t steps, double a, double b, double c, double eps, void* stream) {
  PTO_REQUIRE(batch >= 0 && rows >= 0 && cols >= 0 && steps >= 0,
              "newton_schulz_orthogonalize: negative extent or steps");
  const size_t need = pto_ns5_workspace_bytes(dtype, batch, rows, cols);
  PTO_REQUIRE(need <= pto::kNs5ScratchBytes,
              "newton_schulz_orthogonalize (no-alloc): the call needs " + std::to_string(need) +
                  " bytes of scratch, more than the " + std::to_string(pto::kNs5ScratchBytes) + " it holds");
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ptr = nullptr;
  if (batch * rows * cols != 0 && pto::scratch_ptr(s, &ptr)) return -1;
  pto::ProfSuspend quiet;
  return pto_ns5(G, out, dtype, batch, rows, cols, steps, a, b, c, eps, ptr, pto::kNs5ScratchBytes, stream);
}
