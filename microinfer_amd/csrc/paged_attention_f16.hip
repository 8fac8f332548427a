// Vector paged attention kernels instantiated for F16 caches.
#include "paged_attention_impl.h"

namespace mi {
int32_t launch_vector_f16(const AttnArgs& a, hipStream_t stream) {
  return launch_vector_typed<F16>(a, stream);
}
}  // namespace mi
