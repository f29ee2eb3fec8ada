// MFMA grouped GEMMs for gfx950 (placeholder: not yet enabled).
#include "common.h"
#include "launch.h"

namespace fmoe {

bool gemm_tiled_supported(const GroupedGemmArgs&) { return false; }
bool gemm_stream_supported(const GroupedGemmArgs&) { return false; }
hipError_t launch_gemm_tiled(const GroupedGemmArgs&, hipStream_t) { return hipErrorNotSupported; }
hipError_t launch_gemm_stream(const GroupedGemmArgs&, hipStream_t) { return hipErrorNotSupported; }

}  // namespace fmoe
