/*
 * stlq_mi355 device-buffer helpers.
 *
 * These have no counterpart in the reference: the reference's CUDA providers allocate and copy
 * internally (kernel_provider_cuda_stream_impl.inc). They exist so a caller without its own
 * HIP allocator (a ctypes/FFI binding, a benchmark) can stage inputs in HBM and drive the
 * device-pointer entry point stlq_mi355_encode_device. All calls use the context's device and
 * stream; copies are synchronous with respect to the host.
 */
#ifndef STLQ_MI355_TOOLS_H_
#define STLQ_MI355_TOOLS_H_

#include <stddef.h>
#include <stdint.h>

#include "stlq_mi355.h"

#ifdef __cplusplus
extern "C" {
#endif

int stlq_mi355_dev_alloc(stlq_mi355_ctx* ctx, size_t bytes, void** out);
int stlq_mi355_dev_free(stlq_mi355_ctx* ctx, void* p);
int stlq_mi355_copy_h2d(stlq_mi355_ctx* ctx, void* dst, const void* src, size_t bytes);
int stlq_mi355_copy_d2h(stlq_mi355_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Device-to-device copy by a plain streaming kernel on the context stream (a traffic reference
 * of known size for hardware-counter calibration). bytes must be a multiple of 16. */
int stlq_mi355_dev_copy_kernel(stlq_mi355_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Waits for all work queued on the context stream. */
int stlq_mi355_synchronize(stlq_mi355_ctx* ctx);
/* Device name and compute-unit count of the context's device (name_len bytes incl. NUL). */
int stlq_mi355_device_info(stlq_mi355_ctx* ctx, char* name, int name_len, int* cu_count);

#ifdef __cplusplus
}
#endif

#endif /* STLQ_MI355_TOOLS_H_ */
