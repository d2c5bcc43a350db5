// The GEMV kernels that build faster with the compiler's max-ILP instruction scheduling
// (-mllvm -amdgpu-sched-strategy=max-ilp, set for this file alone by build_lib.py): the
// 8-wave batch-1 kernels, rotated and not, and the 8-wave kernels of batches 2-16 on few row
// tiles per CU (GF4, E2M1 and the native FP4 path; one workgroup per CU), including the ones
// whose waves stage the x of their own spans (kSpanX).  The code is
// fourbit_gemv.hip's; this unit instantiates only those kernels and fb_ilp::launch.
#define FB_GEMV_ILP_TU
#include "fourbit_gemv.hip"
