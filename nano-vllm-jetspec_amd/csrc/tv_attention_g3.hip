// tree_attention_kernel for 3 query heads per KV head (one translation unit per group
// size, so the kernel instantiations compile in parallel).
#include "tv_attention_kernel.h"

namespace tv {

int launch_tree_attention_g3(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s) {
    return launch_group<3>(p, num_items, bf16, exact, s);
}

}  // namespace tv
