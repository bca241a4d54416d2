// Chunked (WY/UT) prefill for gfx950 -- work in progress: the entry point reports
// "not supported" until the MFMA kernels land.
#include "../../include/gdn.h"
#include "gdn_internal.h"

namespace gdn {

hipError_t launch_chunked_prefill(const gdn_layer_args& a, hipStream_t stream) {
  (void)a;
  (void)stream;
  return hipErrorNotSupported;
}

}  // namespace gdn
