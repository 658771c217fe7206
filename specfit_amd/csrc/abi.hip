// Library-level entry points: version, error names, and the expert H2D copy.
#include "sf_common.h"

extern "C" int sf_abi_version(void) { return SF_ABI_VERSION; }

extern "C" const char* sf_error_string(int code) {
  switch (code) {
    case SF_OK:
      return "success";
    case SF_ERR_INVALID_ARGUMENT:
      return "invalid argument";
    case SF_ERR_UNSUPPORTED_SHAPE:
      return "unsupported shape";
    case SF_ERR_MISALIGNED:
      return "misaligned buffer";
    case SF_ERR_TOO_MANY_EXPERTS:
      return "too many experts";
    case SF_ERR_SCRATCH_LIMIT:
      return "workspace exceeds the allocation-free entry point's scratch array";
    default:
      break;
  }
  if (code >= SF_ERR_HIP_BASE) return hipGetErrorString(static_cast<hipError_t>(code - SF_ERR_HIP_BASE));
  return "unknown error";
}

// The copy replaces slot.tensor.copy_(pinned_source, non_blocking=True) of the
// reference cache (src/specfit/runtime/gpu_expert_cache.py:556-561).  From
// page-locked memory hipMemcpyAsync is an SDMA transfer that does not occupy
// compute units, so it overlaps with expert GEMMs on the compute stream.
extern "C" int sf_copy_h2d(void* device_dst, const void* host_src, size_t bytes,
                           sf_stream_t stream) {
  if (bytes == 0) return SF_OK;
  if (!device_dst || !host_src) return SF_ERR_INVALID_ARGUMENT;
  SF_HIP_CHECK(hipMemcpyAsync(device_dst, host_src, bytes, hipMemcpyHostToDevice,
                              reinterpret_cast<hipStream_t>(stream)));
  return SF_OK;
}
