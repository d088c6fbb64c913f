// placeholder, replaced by the chunked prefill kernel
#include "gdn_common.h"
hipError_t gdn_chunk_prefill_launch(const gdn_tensor*, const gdn_tensor*, const gdn_tensor*, const gdn_tensor*,
                                    const gdn_tensor*, gdn_tensor*, const gdn_tensor*, const gdn_tensor*,
                                    gdn_tensor*, float, hipStream_t) {
  return hipErrorNotSupported;
}
