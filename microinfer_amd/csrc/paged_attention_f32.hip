// Vector paged attention kernels instantiated for F32 caches.
#include "paged_attention_impl.h"

namespace mi {
int32_t launch_vector_f32(const AttnArgs& a, hipStream_t stream) {
  return launch_vector_typed<F32>(a, stream);
}
}  // namespace mi
