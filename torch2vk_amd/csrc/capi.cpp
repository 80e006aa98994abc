// Version and status strings of the libt2h C ABI.
#include "t2h.h"

extern "C" int t2h_abi_version(void) { return 1; }

extern "C" const char* t2h_status_string(int status) {
    switch (status) {
        case T2H_OK: return "ok";
        case T2H_ERR_NULL: return "a required pointer is null";
        case T2H_ERR_SHAPE: return "shape violates the kernel contract";
        case T2H_ERR_DTYPE: return "unsupported dtype";
        case T2H_ERR_UNSUPPORTED: return "shape or option not supported by this build";
        case T2H_ERR_ARG: return "invalid argument";
        case T2H_ERR_WORKSPACE: return "workspace too small";
        case T2H_ERR_ALIGN: return "pointer not 16-byte aligned";
        default: return status >= T2H_ERR_HIP_BASE ? "HIP launch error" : "unknown status";
    }
}
