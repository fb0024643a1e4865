/* memory.h - device management and transfers of libgpu_engine.so (gfx950 build).
 *
 * Drop-in replacement for the reference's gpu/cuda/memory.h (lines 11-36),
 * which gpu/bindings/gpu.h:20-68 re-declares for cgo. dtype codes of the copy
 * functions (memory.cu:145-213): 0 = fp32 -> fp32, 1 = fp32 host <-> fp16
 * device (round to nearest even on the way in), 2 = int8. Copies are
 * synchronous with respect to the host, like the reference's cudaMemcpy.
 */
#ifndef NG_MEMORY_H
#define NG_MEMORY_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same layout as memory.h:12-17. major/minor are the gfx IP version (9, 5 on gfx950). */
typedef struct {
    char name[256];
    int major;
    int minor;
    size_t total_memory;
} DeviceInfo;

int cuda_init(int device_id);                 /* memory.h:20 (memory.cu:32-56) */
void cuda_shutdown(void);                     /* memory.h:21 (memory.cu:58-68) */
int cuda_get_device_count(int* count);        /* memory.h:22 (memory.cu:70-73) */
int cuda_set_device(int device_id);           /* memory.h:23 (memory.cu:75-79) */
int cuda_get_device_info(DeviceInfo* info);   /* memory.h:24 (memory.cu:81-92) */
int cuda_sync_device(void);                   /* memory.h:25 (memory.cu:94-97) */
int cuda_get_memory_used(size_t* used);       /* memory.h:26 (memory.cu:99-104) */

int cuda_malloc(void** ptr, size_t size);     /* memory.h:29 (memory.cu:110-117) */
void cuda_free(void* ptr);                    /* memory.h:30 (memory.cu:119-123) */

/* memory.h:33-36 (memory.cu:145-223) */
int cuda_copy_to_device(void* dst, const void* src, size_t num_elements, int dtype);
int cuda_copy_to_host(void* dst, const void* src, size_t num_elements, int dtype);
int cuda_copy_int8_to_device(void* dst, const void* src, size_t num_elements);
int cuda_copy_int8_to_host(void* dst, const void* src, size_t num_elements);

#ifdef __cplusplus
}
#endif

#endif /* NG_MEMORY_H */
