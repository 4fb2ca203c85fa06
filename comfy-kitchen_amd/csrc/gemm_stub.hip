// Placeholder entry points for the GEMMs until their kernels land.
#include "ckh_common.h"

extern "C" int ckh_scaled_mm_mxfp8(const void*, const void*, const void*, const void*, const void*, void*, int64_t,
                                   int64_t, int64_t, int, int, uintptr_t) {
    ckh::set_error("scaled_mm_mxfp8: not implemented in this build");
    return CKH_ERR_INVALID;
}

extern "C" int ckh_scaled_mm_nvfp4(const void*, const void*, const void*, const void*, const void*, const void*,
                                   void*, int64_t, int64_t, int64_t, int, int, uintptr_t) {
    ckh::set_error("scaled_mm_nvfp4: not implemented in this build");
    return CKH_ERR_INVALID;
}
