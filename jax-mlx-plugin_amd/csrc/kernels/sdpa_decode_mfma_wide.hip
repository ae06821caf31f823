// Head sizes 32 and 96 of the MFMA decode: the kernels of
// sdpa_decode_mfma.hip instantiated in a translation unit of their own, so
// they compile in parallel with the 64 / 128 ones.
#define MFX_DECODE_WIDE 1
#include "sdpa_decode_mfma.hip"
