// The scaled-key-path instantiations of attn_fwd_kernel (attention_kernel.hpp),
// in a translation unit of their own so that the build can compile them with
// their own machine scheduler: LLVM's iterative ILP scheduler orders this
// path's tile loop 1.0-1.5% faster at the long-sequence shape (same-box A/B),
// while the plain path keeps the max-memory-clause scheduler, which suits it
// better at short sequences.  attention_fwd.hip launches them through
// scaled_path_kernel().

#include "attention_kernel.hpp"

namespace sah {
namespace {

template <typename T, int WAVES>
const void* scaled_kernel(int qg, int num_stages) {
  if (qg == 1)
    return num_stages == 2 ? reinterpret_cast<const void*>(&attn_fwd_kernel<T, 1, 2, WAVES, kPathScaled>)
                           : reinterpret_cast<const void*>(&attn_fwd_kernel<T, 1, 1, WAVES, kPathScaled>);
  return num_stages == 2 ? reinterpret_cast<const void*>(&attn_fwd_kernel<T, 2, 2, WAVES, kPathScaled>)
                         : reinterpret_cast<const void*>(&attn_fwd_kernel<T, 2, 1, WAVES, kPathScaled>);
}

}  // namespace

const void* scaled_path_kernel(bool bf16_type, int waves, int qg, int num_stages) {
  if (bf16_type)
    return waves == 8 ? scaled_kernel<bf16, 8>(qg, num_stages) : scaled_kernel<bf16, 4>(qg, num_stages);
  return waves == 8 ? scaled_kernel<f16, 8>(qg, num_stages) : scaled_kernel<f16, 4>(qg, num_stages);
}

}  // namespace sah
