// MFMA paged-decode kernel for bf16 / e4m3fn caches (gfx950).
#include "cf_device.hpp"
#include "cf_host.hpp"
#include "decode_params.hpp"

namespace cf {

bool decode_mfma_supported(const DecodeParams&, int, int) { return false; }

int32_t launch_decode_mfma(const DecodeParams&, int, int, hipStream_t) {
  set_error("MFMA decode path not available");
  return CF_ERR_UNSUPPORTED;
}

}  // namespace cf
