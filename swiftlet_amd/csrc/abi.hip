// Library-level C ABI: status names, version, device presence.
#include "internal.hpp"

extern "C" const char *swq_strerror(int status) {
    switch (status) {
        case SWQ_OK: return "ok";
        case SWQ_ERR_INVALID_ARGUMENT: return "invalid argument";
        case SWQ_ERR_BAD_SHAPE: return "bad shape (in_dim % group_size, group_size % codes per word, or dims)";
        case SWQ_ERR_UNSUPPORTED_BITS: return "unsupported bits";
        case SWQ_ERR_UNSUPPORTED_DTYPE: return "unsupported dtype";
        case SWQ_ERR_MISALIGNED: return "misaligned pointer or offset";
        case SWQ_ERR_WORKSPACE: return "workspace missing or too small";
        case SWQ_ERR_EXPERT_RANGE: return "top_k outside [1, num_experts]";
        case SWQ_ERR_HIP: return "HIP runtime error";
        case SWQ_ERR_NO_DEVICE: return "no HIP device";
        case SWQ_ERR_LIMIT: return "size above compiled limit";
        case SWQ_ERR_MISSING_TENSOR: return "tensor or section not found";
        case SWQ_ERR_IO: return "file open or read failed";
        case SWQ_ERR_FORMAT: return "malformed checkpoint, JSON or qpack layout";
        case SWQ_ERR_STALLED:
            return "a single-launch MoE call ran out of a bounded wait (workgroups not co-resident); its outputs are invalid";
        default: return "unknown status";
    }
}

extern "C" int swq_version(void) { return 100; }

extern "C" int swq_device_count(int *count) {
    if (!count) return SWQ_ERR_INVALID_ARGUMENT;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        *count = 0;
        return SWQ_ERR_NO_DEVICE;
    }
    *count = n;
    return SWQ_OK;
}
