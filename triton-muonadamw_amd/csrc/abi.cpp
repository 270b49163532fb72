// Version and status-text entry points of the C ABI (host only).
#include "muonadamw_amd.h"

#include <hip/hip_runtime_api.h>

extern "C" int mamw_abi_version(void) { return MAMW_ABI_VERSION; }

extern "C" const char* mamw_strerror(int status) {
    switch (status) {
        case MAMW_OK: return "success";
        case MAMW_ERR_NULL: return "a required pointer is NULL";
        case MAMW_ERR_COUNT: return "tensor or matrix count out of range";
        case MAMW_ERR_NUMEL: return "element count negative or beyond the supported size";
        case MAMW_ERR_SHAPE: return "rows/cols out of range or not equal within one call";
        case MAMW_ERR_ALIGN: return "pointer misaligned for its element type";
        case MAMW_ERR_WORKSPACE: return "workspace NULL, not 256-byte aligned or too small";
        case MAMW_ERR_HYPER: return "hyper-parameter out of range";
        case MAMW_ERR_TABLE: return "host table buffer too small";
        case MAMW_ERR_ALIAS: return "buffers that must be distinct overlap";
        case MAMW_ERR_SCRATCH:
            return "the step needs more workspace than the library's static scratch (MAMW_NOALLOC_SCRATCH_BYTES)";
        default: break;
    }
    if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
    return "unknown status";
}
