// Single gfx950 code object holding every kernel of the quantized-matmul
// backend. Built with `hipcc --genco --offload-arch=gfx950` and embedded in
// libqmm.so; the host side loads it with hipModuleLoadData and launches the
// kernels by name with hipModuleLaunchKernel.
#include "qmm_common.h"
#include "qmm_quant_kernels.h"
#include "qmm_gemv_kernels.h"
#include "qmm_gemv1p_kernels.h"
#include "qmm_mmq_kernels.h"
#include "qmm_moe_kernels.h"
#include "qmm_gemvm_kernels.h"
#include "qmm_decode_kernels.h"
#include "qmm_calib_kernels.h"
