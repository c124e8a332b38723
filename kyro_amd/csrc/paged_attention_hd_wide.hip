// The bf16 MFMA attention kernel at head dims 112, 160, 192 and 224: the kernels of
// paged_attention.hip, instantiated in a translation unit of their own so that these instances
// compile in parallel with the other head dims'.
#define KYRO_ATTN_HD_UNIT 2
#include "paged_attention.hip"
