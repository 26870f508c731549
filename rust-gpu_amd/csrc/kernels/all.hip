// all.hip -- the single translation unit that becomes the library's gfx950
// code object (t0_kernels.hsaco, embedded into libt0gpu.so).
#include "gemm_bf16.hip"
#include "w4a16.hip"
#include "aux.hip"
