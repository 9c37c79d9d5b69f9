// fp16 instances of the block-sparse attention forward (gfx950): the same
// kernels as the bf16 ones (bsa_kernel.h) on v_mfma_f32_32x32x16_f16, built in
// a translation unit of their own so the two element types compile in
// parallel.
#include "bsa_kernel.h"

int bsa_launch_f16(bsa::BsaParams p, float* part, int64_t part_groups, hipStream_t stream,
                   const char* who) {
  return bsa::launch_typed<_Float16>(p, part, part_groups, stream, who);
}
