/* The header is plain C: this translation unit only has to compile. */
#include "mi_sdvk.h"

int use_header(void) {
    mi_attn_args a = {0};
    mi_block_dims d = {0};
    mi_gguf_tensor_info t;
    (void)t;
    return (int)sizeof a + (int)sizeof d + MI_ERR_NOT_FOUND;
}
