// tq_abi.hip -- version and status helpers of the libtq C ABI.
#include "tq_common.h"

extern "C" int tq_abi_version(void) { return TQ_ABI_VERSION; }

extern "C" const char* tq_status_string(int status) {
    switch (status) {
        case TQ_OK: return "ok";
        case TQ_ERR_INVALID_ARGUMENT: return "invalid argument";
        case TQ_ERR_UNSUPPORTED: return "unsupported shape, alignment or bit width";
        case TQ_ERR_WORKSPACE: return "workspace missing or too small";
        case TQ_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}
