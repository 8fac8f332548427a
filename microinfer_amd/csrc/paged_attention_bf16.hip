// Vector paged attention kernels instantiated for BF16 caches.
#include "paged_attention_impl.h"

namespace mi {
int32_t launch_vector_bf16(const AttnArgs& a, hipStream_t stream) {
  return launch_vector_typed<BF16>(a, stream);
}
}  // namespace mi
