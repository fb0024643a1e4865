/* stream.h - process-global launch stream of libgpu_engine.so (gfx950 build).
 *
 * Drop-in replacement for the reference's gpu/cuda/stream.h (lines 14-17,
 * defined in stream.cu:4-12). Every kernel of this library is enqueued on the
 * stream returned by ng_get_stream(); NULL (the default) is the null stream.
 * A caller that captures a HIP graph sets its capture stream here first.
 * The stream is stored per process, not per thread, as in the reference.
 */
#ifndef NG_STREAM_H
#define NG_STREAM_H

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

hipStream_t ng_get_stream(void);
void ng_set_stream(hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NG_STREAM_H */
