/* attn_devutil.c -- device plumbing for tests and the benchmark (see attn_devutil.h). */
#define __HIP_PLATFORM_AMD__ 1
#include "attn_devutil.h"
#include "attn_flash.h"

#include <hip/hip_runtime_api.h>
#include <string.h>

int attn_dev_count(int *n) { return (int)hipGetDeviceCount(n); }
int attn_dev_malloc(void **p, size_t bytes) { return (int)hipMalloc(p, bytes); }
int attn_dev_free(void *p) { return (int)hipFree(p); }
int attn_dev_memcpy_htod(void *dst, const void *src, size_t bytes) {
    return (int)hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
}
int attn_dev_memcpy_dtoh(void *dst, const void *src, size_t bytes) {
    return (int)hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
}
int attn_dev_memcpy_dtod(void *dst, const void *src, size_t bytes) {
    return (int)hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice);
}
int attn_dev_memset(void *dst, int value, size_t bytes) {
    return (int)hipMemset(dst, value, bytes);
}
int attn_dev_synchronize(void) { return (int)hipDeviceSynchronize(); }

int attn_dev_info(char *name, size_t name_len, char *arch, size_t arch_len, int *cus,
                  int *clock_khz, int *l2_bytes) {
    hipDeviceProp_t p;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return (int)e;
    e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess)
        return (int)e;
    if (name && name_len) {
        strncpy(name, p.name, name_len - 1);
        name[name_len - 1] = 0;
    }
    if (arch && arch_len) {
        strncpy(arch, p.gcnArchName, arch_len - 1);
        arch[arch_len - 1] = 0;
    }
    if (cus)
        *cus = p.multiProcessorCount;
    if (clock_khz)
        *clock_khz = p.clockRate;
    if (l2_bytes)
        *l2_bytes = p.l2CacheSize;
    return 0;
}

int attn_dev_event_create(void **ev) { return (int)hipEventCreate((hipEvent_t *)ev); }
int attn_dev_event_destroy(void *ev) { return (int)hipEventDestroy((hipEvent_t)ev); }
int attn_dev_event_record(void *ev) {
    return (int)hipEventRecord((hipEvent_t)ev, (hipStream_t)attn_flash_get_stream());
}
int attn_dev_event_elapsed_ms(void *start, void *stop, float *ms) {
    hipError_t e = hipEventSynchronize((hipEvent_t)stop);
    if (e != hipSuccess)
        return (int)e;
    return (int)hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop);
}
