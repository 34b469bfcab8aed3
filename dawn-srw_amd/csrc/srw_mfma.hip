// srw_mfma.hip -- MFMA kernel family (placeholder until the tiled kernels land).
#include "srw_internal.hpp"

namespace srw {

size_t mfma_workspace_bytes(const srw_desc_t&) { return 0; }
bool mfma_supports(const srw_desc_t&) { return false; }
hipError_t mfma_forward(const LaunchArgs&, const char** path_name) {
  *path_name = "mfma";
  return hipErrorNotSupported;
}

}  // namespace srw
