/* Kernel-level C-ABI (include/lunelette_kernels.h): argument checks and launch
 * of single operators, device plumbing for callers without another HIP
 * binding, and the shared thread-local diagnostic. */
#include "lunelette_kernels.h"
#include "lh_internal.h"

#include <stdarg.h>
#include <stdatomic.h>
#include <stdio.h>

static _Thread_local char last_error[512];

void lh_set_error(const char *format, ...)
{
    va_list args;
    va_start(args, format);
    vsnprintf(last_error, sizeof last_error, format, args);
    va_end(args);
}

const char *lh_last_error(void)
{
    return last_error;
}

static int ok(hipError_t status, const char *what)
{
    if (status != hipSuccess) {
        lh_set_error("%s: %s", what, hipGetErrorString(status));
        return -1;
    }
    return 0;
}

static atomic_uint allocation_fail_at;  /* 1-based allocation to fail; 0 never */
static atomic_uint allocation_count;    /* allocations since the counter was armed */
static atomic_long allocation_live;     /* allocations not yet freed */

void lh_allocations_arm(unsigned nth)
{
    atomic_store_explicit(&allocation_count, 0, memory_order_relaxed);
    atomic_store_explicit(&allocation_fail_at, nth, memory_order_relaxed);
}

unsigned lh_allocations_count(void)
{
    return atomic_load_explicit(&allocation_count, memory_order_relaxed);
}

long lh_allocations_live(void)
{
    return atomic_load_explicit(&allocation_live, memory_order_relaxed);
}

static int forced_failure(void)
{
    unsigned n = atomic_fetch_add_explicit(&allocation_count, 1, memory_order_relaxed) + 1;
    unsigned at = atomic_load_explicit(&allocation_fail_at, memory_order_relaxed);
    return at && n == at;
}

static void count_live(long delta)
{
    atomic_fetch_add_explicit(&allocation_live, delta, memory_order_relaxed);
}

hipError_t lh_dev_malloc(void **ptr, size_t bytes)
{
    *ptr = NULL;
    if (forced_failure()) {
        return hipErrorOutOfMemory;
    }
    hipError_t status = hipMalloc(ptr, bytes ? bytes : 16);
    if (status == hipSuccess) {
        count_live(1);
    } else {
        *ptr = NULL;
    }
    return status;
}

hipError_t lh_host_malloc(void **ptr, size_t bytes, unsigned flags)
{
    *ptr = NULL;
    if (forced_failure()) {
        return hipErrorOutOfMemory;
    }
    hipError_t status = hipHostMalloc(ptr, bytes ? bytes : 16, flags);
    if (status == hipSuccess) {
        count_live(1);
    } else {
        *ptr = NULL;
    }
    return status;
}

void lh_dev_free(void *ptr)
{
    if (ptr) {
        (void)hipFree(ptr);
        count_live(-1);
    }
}

void lh_host_free(void *ptr)
{
    if (ptr) {
        (void)hipHostFree(ptr);
        count_live(-1);
    }
}

int lh_device_count(void)
{
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess ? n : 0;
}

void *lh_device_alloc(size_t bytes)
{
    void *p = NULL;
    return ok(lh_dev_malloc(&p, bytes), "hipMalloc") ? NULL : p;
}

void lh_device_free(void *d_ptr)
{
    lh_dev_free(d_ptr);
}

void *lh_host_alloc_pinned(size_t bytes)
{
    void *p = NULL;
    return ok(lh_host_malloc(&p, bytes, hipHostMallocDefault), "hipHostMalloc") ? NULL : p;
}

void lh_host_free_pinned(void *ptr)
{
    lh_host_free(ptr);
}

int lh_memcpy_htod(void *d_dst, const void *src, size_t bytes)
{
    return ok(hipMemcpy(d_dst, src, bytes, hipMemcpyHostToDevice), "copy to device");
}

int lh_memcpy_dtoh(void *dst, const void *d_src, size_t bytes)
{
    return ok(hipMemcpy(dst, d_src, bytes, hipMemcpyDeviceToHost), "copy to host");
}

int lh_memcpy_dtod(void *d_dst, const void *d_src, size_t bytes)
{
    return ok(hipMemcpy(d_dst, d_src, bytes, hipMemcpyDeviceToDevice), "device copy");
}

int lh_memset_device(void *d_dst, int value, size_t bytes)
{
    return ok(hipMemset(d_dst, value, bytes), "device memset");
}

int lh_device_synchronize(void)
{
    return ok(hipDeviceSynchronize(), "device synchronize");
}

void *lh_stream_create(void)
{
    hipStream_t s = NULL;
    return ok(hipStreamCreate(&s), "stream create") ? NULL : (void *)s;
}

int lh_stream_synchronize(void *stream)
{
    return ok(hipStreamSynchronize((hipStream_t)stream), "stream synchronize");
}

void lh_stream_destroy(void *stream)
{
    if (stream) {
        (void)hipStreamDestroy((hipStream_t)stream);
    }
}

void *lh_event_create(void)
{
    hipEvent_t e = NULL;
    return ok(hipEventCreate(&e), "event create") ? NULL : (void *)e;
}

int lh_event_record(void *event, void *stream)
{
    return ok(hipEventRecord((hipEvent_t)event, (hipStream_t)stream), "event record");
}

int lh_event_elapsed_ms(void *start, void *stop, float *milliseconds)
{
    if (ok(hipEventSynchronize((hipEvent_t)stop), "event synchronize")) {
        return -1;
    }
    return ok(hipEventElapsedTime(milliseconds, (hipEvent_t)start, (hipEvent_t)stop),
        "event elapsed");
}

void lh_event_destroy(void *event)
{
    if (event) {
        (void)hipEventDestroy((hipEvent_t)event);
    }
}

static int launched(int status, const char *what)
{
    if (status) {
        lh_set_error("%s launch failed: %s", what, hipGetErrorString(hipGetLastError()));
        return -1;
    }
    return 0;
}

static int shape_ok(const void *w, const void *x, const void *y, size_t rows, size_t cols,
    size_t tokens)
{
    if (!w || !x || !y || !rows || !cols || !tokens || rows > 0x7fffffffu || cols > 0x7fffffffu ||
        tokens > 65535) {
        lh_set_error("matvec: require pointers, rows/cols in 1..2^31-1, tokens in 1..65535");
        return 0;
    }
    return 1;
}

int lh_fp8_matvec(const uint8_t *d_w, float scale, const float *d_x, float *d_y, size_t rows,
    size_t cols, size_t tokens, int lookup, void *stream)
{
    if (!shape_ok(d_w, d_x, d_y, rows, cols, tokens)) {
        return -1;
    }
    return launched(lh_launch_matvec(0, lookup != 0, d_w, scale, d_x, d_y, NULL, (uint32_t)rows,
        (uint32_t)cols, (uint32_t)tokens, (hipStream_t)stream), "fp8 matvec");
}

int lh_f32_matvec(const float *d_w, const float *d_x, float *d_y, size_t rows, size_t cols,
    size_t tokens, void *stream)
{
    if (!shape_ok(d_w, d_x, d_y, rows, cols, tokens)) {
        return -1;
    }
    return launched(lh_launch_matvec(2, 0, d_w, 1.0f, d_x, d_y, NULL, (uint32_t)rows,
        (uint32_t)cols, (uint32_t)tokens, (hipStream_t)stream), "f32 matvec");
}

int lh_bf16_matvec(const uint16_t *d_w, const float *d_x, float *d_y, size_t rows, size_t cols,
    size_t tokens, void *stream)
{
    if (!shape_ok(d_w, d_x, d_y, rows, cols, tokens)) {
        return -1;
    }
    return launched(lh_launch_matvec(1, 0, d_w, 1.0f, d_x, d_y, NULL, (uint32_t)rows,
        (uint32_t)cols, (uint32_t)tokens, (hipStream_t)stream), "bf16 matvec");
}

int lh_rmsnorm(const float *d_gamma, const float *d_x, float *d_out, size_t width, size_t tokens,
    void *stream)
{
    if (!d_gamma || !d_x || !d_out || !width || width > 16384 || !tokens || tokens > 0x7fffffffu) {
        lh_set_error("rmsnorm: require pointers, width 1..16384, tokens >= 1");
        return -1;
    }
    return launched(lh_launch_rmsnorm(d_gamma, d_x, d_out, (uint32_t)width, (uint32_t)tokens,
        (hipStream_t)stream), "rmsnorm");
}

int lh_element(int mode, const float *d_first, const float *d_second, float *d_out, size_t n,
    void *stream)
{
    if (mode < 0 || mode > 2 || !d_first || !d_out || (mode != 1 && !d_second) || !n ||
        n > ((size_t)1 << 40)) {
        lh_set_error("element: mode 0 add, 1 SiLU, 2 multiply; pointers and n required");
        return -1;
    }
    return launched(lh_launch_element(mode, d_first, d_second, d_out, n, (hipStream_t)stream),
        "element");
}

int lh_read_floor(const void *d_src, size_t bytes, unsigned grid, unsigned unroll,
    unsigned *d_sink, void *stream)
{
    const size_t unit = (size_t)grid * 4 * 64 * 16 * unroll;
    if (!d_src || !d_sink || !grid || grid > 65536 ||
        (unroll != 1 && unroll != 2 && unroll != 4 && unroll != 8) || !bytes ||
        bytes % unit) {
        lh_set_error("read_floor: pointers, grid 1..65536, unroll 1/2/4/8 and bytes a multiple "
            "of grid*4*64*16*unroll required");
        return -1;
    }
    return launched(lh_launch_read_floor(d_src, bytes, grid, unroll, d_sink,
        (hipStream_t)stream), "read floor");
}

int lh_rope(const float *d_x, const float *d_cos, const float *d_sin, const float *d_qfactor,
    float *d_out, size_t width, size_t tokens, void *stream)
{
    if (!d_x || !d_cos || !d_sin || !d_out || !width || width % 128 || !tokens ||
        width * tokens > 0xffffffffu) {
        lh_set_error("rope: width must be a positive multiple of 128");
        return -1;
    }
    return launched(lh_launch_rope(d_x, d_cos, d_sin, d_qfactor, d_out, (uint32_t)width,
        (uint32_t)tokens, (hipStream_t)stream), "rope");
}

int lh_fp8_decode(const uint8_t *d_codes, float *d_out, size_t n, void *stream)
{
    if (!d_codes || !d_out || !n) {
        lh_set_error("fp8_decode: pointers and n required");
        return -1;
    }
    return launched(lh_launch_fp8_decode(d_codes, d_out, n, (hipStream_t)stream), "fp8 decode");
}

int lh_expf(const float *d_x, float *d_out, size_t n, void *stream)
{
    if (!d_x || !d_out || !n) {
        lh_set_error("expf: pointers and n required");
        return -1;
    }
    return launched(lh_launch_expf(d_x, d_out, n, (hipStream_t)stream), "expf");
}
