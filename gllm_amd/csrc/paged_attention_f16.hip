// fp16 instantiations of the paged / dense attention kernels: the same source
// as paged_attention.hip with the element type fixed to _Float16, built as its
// own unit (the bf16 unit dispatches to launch_paged_f16 / launch_dense_f16).
#define GLLM_PAGED_F16 1
#include "paged_attention.hip"
