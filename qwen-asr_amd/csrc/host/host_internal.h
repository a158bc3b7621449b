/* host_internal.h - helpers shared by the C host files of the library. */
#ifndef QK_HOST_INTERNAL_H
#define QK_HOST_INTERNAL_H

#include "qwen_asr_hip.h"
#include "../kernels/qk_kernels.h"

#include <stdio.h>

/* Record the message returned by qwen_hip_last_error() (thread local). */
void qk_set_err(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

#define QK_HIP(call)                                                            \
    do {                                                                        \
        hipError_t e__ = (call);                                                \
        if (e__ != hipSuccess) {                                                \
            qk_set_err("%s:%d %s: %s", __FILE__, __LINE__, #call,               \
                       hipGetErrorString(e__));                                 \
            return QWEN_HIP_EDEVICE;                                            \
        }                                                                       \
    } while (0)

#define QK_TRY(expr)                                                            \
    do {                                                                        \
        int r__ = (expr);                                                       \
        if (r__ != 0) {                                                         \
            if (r__ == QWEN_HIP_EINVAL)                                         \
                qk_set_err("%s:%d launch rejected its arguments: %s",           \
                           __FILE__, __LINE__, #expr);                          \
            else if (r__ == QWEN_HIP_EDEVICE)                                   \
                qk_set_err("%s:%d launch failed: %s", __FILE__, __LINE__,       \
                           #expr);                                              \
            return r__;                                                         \
        }                                                                       \
    } while (0)

#endif
