// noalloc.hip - qwen_hip_linear_nobias_bf16_noalloc: the op-level linear
// (qwen_asr_kernels.h:41-42 semantics, like qwen_hip_linear_nobias_bf16) for
// callers that cannot allocate device memory: code being captured into a HIP
// graph, tight serving loops, harnesses that forbid hipMalloc.
//
// The seq > 1 product needs temporary device memory (the bf16 hi/lo split of x
// and, for small tile grids, the split-K partials).  Here it lives in one
// file-scope device array of QK_NOALLOC_SCRATCH_BYTES that every GPU the
// library runs on holds from module load until the process ends.  In host code
// the array's name is only a stand-in: its device address is taken once per
// device with hipGetSymbolAddress (on the device's first call, with that device
// current) and only that address is ever handed to kernels.
//
// The entry point enqueues its kernels on the caller's stream and returns
// without synchronising, allocating or freeing anything.  Every call on one
// GPU uses that GPU's same array, which keeps the last call's contents (every
// byte a call reads it has written first, so nothing needs clearing): calls
// whose kernels overlap in time on one GPU race on it, so a caller orders them
// (one stream, or events).
#include "common.h"
#include "qk_kernels.h"
#include "qwen_asr_hip.h"

#include <pthread.h>

#define QK_NOALLOC_SCRATCH_BYTES (32u << 20)
#define QK_NOALLOC_MAX_DEVICES 64

static __device__ __align__(256) unsigned char scratch[QK_NOALLOC_SCRATCH_BYTES];

static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;
static void *g_scratch[QK_NOALLOC_MAX_DEVICES];

extern "C" void qk_set_err(const char *fmt, ...);

// Device address of `scratch` on the current device (looked up once per device).
static int scratch_ptr(void **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= QK_NOALLOC_MAX_DEVICES) {
        qk_set_err("linear_noalloc: no usable current device");
        return QWEN_HIP_EDEVICE;
    }
    pthread_mutex_lock(&g_lock);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            pthread_mutex_unlock(&g_lock);
            qk_set_err("linear_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
            return QWEN_HIP_EDEVICE;
        }
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    pthread_mutex_unlock(&g_lock);
    return 0;
}

extern "C" size_t qwen_hip_linear_noalloc_max_bytes(void) { return QK_NOALLOC_SCRATCH_BYTES; }

extern "C" int qwen_hip_linear_nobias_bf16_noalloc(float *y, const float *x, const uint16_t *W, int seq, int in_dim,
                                                   int out_dim, hipStream_t s) {
    if (!y || !x || !W || seq <= 0 || in_dim <= 0 || out_dim <= 0) {
        qk_set_err("linear_noalloc: bad argument");
        return QWEN_HIP_EINVAL;
    }
    if (seq == 1) {   // the GEMV needs no temporary memory
        qk_gemv_args g = {};
        g.W = W;
        g.rows = out_dim;
        g.K = in_dim;
        g.x = x;
        g.y = y;
        g.epi = QK_EPI_STORE;
        return qk_gemv_launch(&g, s);
    }
    const size_t need = qk_linear_ws_bytes(seq, in_dim, out_dim);
    if (need > QK_NOALLOC_SCRATCH_BYTES) {
        qk_set_err("linear_noalloc: seq %d x in %d x out %d needs %zu bytes of scratch, more than the %u available",
                   seq, in_dim, out_dim, need, QK_NOALLOC_SCRATCH_BYTES);
        return QWEN_HIP_EINVAL;
    }
    void *ws = nullptr;
    int rc = scratch_ptr(&ws);
    if (rc) return rc;
    return qk_linear_gemm(y, x, W, seq, in_dim, out_dim, ws, s);
}
