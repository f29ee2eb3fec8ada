// Device-resident scratch of fmoe_moe_ffn_block_noalloc: the block's
// workspace (routing ids and weights, permutation, decode-router partials,
// SwiGLU rows h, fp32 per-slot outputs y) carved from one file-scope device
// array instead of caller- or library-allocated memory, for callers that
// cannot allocate (code under HIP graph capture, serving loops, harnesses
// that forbid hipMalloc).
//
// Every GPU the library runs on holds its own copy of the array, at its own
// address, until the process ends.  Host code never passes the array's name
// to a kernel (in host code it names a host-side stand-in, not device
// memory): the device address comes from hipGetSymbolAddress, looked up once
// per device with that device current, and is cached per device ordinal.
#include "common.h"
#include "fmoe.h"
#include "launch.h"

#include <mutex>

namespace fmoe {
namespace {

static_assert(FMOE_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size must keep 256-byte alignment");

static __device__ __align__(256) unsigned char scratch[FMOE_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {nullptr};

}  // namespace

hipError_t noalloc_scratch(int device, void** ptr) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_ptr[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p || reinterpret_cast<uintptr_t>(p) % 256) return hipErrorInvalidValue;
    g_ptr[device] = p;
  }
  *ptr = g_ptr[device];
  return hipSuccess;
}

}  // namespace fmoe
