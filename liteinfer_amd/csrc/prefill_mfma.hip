// Packed / chunked prefill on CDNA4 matrix cores.
#include "li_attention.h"

namespace li {

bool prefill_mfma_applies(const AttnArgs&, int) { return false; }

int launch_prefill_mfma(const AttnArgs&, int, hipStream_t) {
  return fail(LI_EUNSUPPORTED, "prefill MFMA kernel is not built");
}

}  // namespace li
