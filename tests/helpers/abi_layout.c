/* Prints the sizes and offsets of the device-backend ABI structs in the format of
 * hymt2_hip_abi_layout(). Built twice by tests/test_abi.py: against include/hymt2_hip.h, and
 * (with -DFROM_REFERENCE and the reference's src/ on the include path) against the reference's
 * own declarations in src/internal.h and src/device.h. */
#include <stddef.h>
#include <stdio.h>

#ifdef FROM_REFERENCE
#include "internal.h"
#include "device.h"
typedef weight_t W;
typedef hy_fused_layer FL;
typedef hy_fused_args FA;
typedef hy_device_ops OPS;
typedef q8k_block Q8K;
#else
#include "hymt2_hip.h"
typedef hymt2_weight W;
typedef hymt2_fused_layer FL;
typedef hymt2_fused_args FA;
typedef hymt2_device_ops OPS;
typedef hymt2_q8k_block Q8K;
#endif

int main(void) {
    printf("weight_t=%zu weight_t.row_bytes=%zu weight_t.pk=%zu weight_t.gpu=%zu hy_fused_layer=%zu "
           "hy_fused_args=%zu hy_fused_args.eps=%zu hy_fused_args.layers=%zu hy_fused_args.logits=%zu "
           "hy_device_ops=%zu q8k_block=%zu\n",
           sizeof(W), offsetof(W, row_bytes), offsetof(W, pk), offsetof(W, gpu), sizeof(FL), sizeof(FA),
           offsetof(FA, eps), offsetof(FA, layers), offsetof(FA, logits), sizeof(OPS), sizeof(Q8K));
    return 0;
}
