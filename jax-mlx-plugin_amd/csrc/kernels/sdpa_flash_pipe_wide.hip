// Head sizes 32 and 96 of the pipelined flash kernel: the kernel of
// sdpa_flash_bf16_pipe.hip instantiated in a translation unit of its own, so
// these instantiations compile in parallel with the 64 / 128 ones.  (The
// phase-timer instrumentation covers the 64 / 128 kernels only.)
#undef MFX_PHASE_TIMERS
#define MFX_PIPE_WIDE 1
#include "sdpa_flash_bf16_pipe.hip"
