// gemm.hip — prefill dequant-GEMM on the MFMA units (see include/yule_hip.h,
// yule_hip_quantized_gemm).  Not implemented yet: the entry point validates
// its arguments and reports YULE_ERR_UNSUPPORTED.
#include "internal.h"

extern "C" int yule_hip_quantized_gemm(yule_hip_backend *be, yule_buffer, yule_buffer, yule_buffer, uint32_t,
                                       uint32_t, uint32_t, uint32_t) {
    if (!be) return yule::set_error(YULE_ERR_INVALID, "null backend");
    return yule::set_error(YULE_ERR_UNSUPPORTED, "quantized_gemm: not implemented yet");
}
