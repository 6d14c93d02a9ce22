// f16_skinny.hip -- placeholder registration hook (skinny kernels are added
// in a later file revision).
#include "vk_internal.hpp"
namespace vk {
void register_f16_skinny() {}
}  // namespace vk
