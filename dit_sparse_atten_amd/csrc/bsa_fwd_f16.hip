// fp16 instances of the block-sparse attention forward (gfx950): the same
// kernels as the bf16 ones (bsa_kernel.h) on v_mfma_f32_32x32x16_f16, built in
// a translation unit of their own so the two element types compile in
// parallel.
#include "bsa_kernel.h"

int bsa_launch_f16(bsa::BsaParams p, void* scratch, size_t scratch_bytes, hipStream_t stream,
                   const char* who) {
  return bsa::launch_typed<_Float16>(p, scratch, scratch_bytes, stream, who);
}
