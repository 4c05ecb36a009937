// tree_attention_kernel at head size 256 for 1 query heads per KV head (one translation unit
// per instance group, so the instantiations compile in parallel).
#include "tv_attention_kernel.h"

namespace tv {

int launch_tree_attention_d256_g1(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s) {
    return launch_group<1, 256>(p, num_items, bf16, exact, s);
}

}  // namespace tv
