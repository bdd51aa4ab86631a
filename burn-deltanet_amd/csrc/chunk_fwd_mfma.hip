// MFMA (bf16) chunk forward — placeholder until the tiled kernels land.
#include "dn_common.hpp"

namespace dn {

bool mfma_fwd_supported(const Dims&, int, int) { return false; }
size_t mfma_fwd_workspace(const Dims&) { return 0; }
hipError_t mfma_fwd(const Dims&, int, const void*, const void*, const void*, const float*,
                    const float*, const float*, const float*, void*, float*, void*,
                    hipStream_t) {
  return hipErrorNotSupported;
}

}  // namespace dn
