// The bf16 MFMA attention kernel at head dims 64, 80, 96 and 256: the kernels of
// paged_attention.hip, instantiated in a translation unit of their own so that these instances
// compile in parallel with the head-dim-128 and vector ones.
#define KYRO_ATTN_HD_UNIT 1
#include "paged_attention.hip"
