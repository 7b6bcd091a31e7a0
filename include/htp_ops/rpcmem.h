/*
 * Shared tensor memory.  Callers of the reference allocate every tensor with
 * rpcmem_alloc, turn it into an fd with rpcmem_to_fd and map it for the
 * executor with fastrpc_mmap (reference src/host/test.c:69-97); requests then
 * name tensors as {fd, offset}.  This library provides the same four calls
 * (Qualcomm libcdsprpc names and signatures) so such callers link unchanged:
 *
 *   rpcmem_alloc   -> pinned host memory (hipHostMalloc) + an fd in the registry;
 *                     the executor keeps a device mirror and copies per request.
 *   rpcmem_to_fd   -> the registry fd of an allocation (-1 if unknown).
 *   fastrpc_mmap   -> makes an fd visible to the executor (unmapped fds fail
 *                     with -2 like reference src/dsp/op_executor.cc:328).
 *   fastrpc_munmap / rpcmem_free -> drop visibility / storage and every cached
 *                     prepacked weight derived from the fd.
 *
 * MI355X extension: RPCMEM_FLAG_AMD_DEVICE allocates the tensor directly in
 * HBM.  The returned pointer is then a device address (not dereferenceable on
 * the host); fill and read it with htp_ops_amd_buffer_write/_read.  Requests on
 * such fds run with no host<->device copies.
 */
#ifndef HTP_OPS_RPCMEM_H
#define HTP_OPS_RPCMEM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RPCMEM_HEAP_ID_SYSTEM 25
#define RPCMEM_DEFAULT_HEAP (-1)
#define RPCMEM_FLAG_UNCACHED 0u
#define RPCMEM_FLAG_CACHED 1u
#define RPCMEM_DEFAULT_FLAGS 1u
#define RPCMEM_FLAG_AMD_DEVICE (1u << 30)

#define FASTRPC_MAP_FD 2
#define CDSP_DOMAIN_ID 3

void rpcmem_init(void);
void rpcmem_deinit(void);
void *rpcmem_alloc(int heapid, uint32_t flags, int size);
void *rpcmem_alloc2(int heapid, uint32_t flags, size_t size);
void rpcmem_free(void *po);
int rpcmem_to_fd(void *po);

int fastrpc_mmap(int domain, int fd, void *addr, int offset, size_t length, int flags);
int fastrpc_munmap(int domain, int fd, void *addr, size_t length);

/* ---- MI355X extensions (no reference counterpart) ------------------------ */

/* Byte size of a registered fd, or -1. */
int64_t htp_ops_amd_buffer_size(int fd);
/* 1 if the fd lives in HBM (RPCMEM_FLAG_AMD_DEVICE), 0 if host, -1 if unknown. */
int htp_ops_amd_buffer_is_device(int fd);
/* Device address of the fd's storage (HBM buffer or the host buffer's mirror),
 * creating the mirror if needed; NULL on error. */
void *htp_ops_amd_buffer_device_ptr(int fd);
/* Synchronous copies between host memory and [offset, offset+bytes) of an fd. */
int htp_ops_amd_buffer_write(int fd, size_t offset, const void *src, size_t bytes);
int htp_ops_amd_buffer_read(int fd, size_t offset, void *dst, size_t bytes);
/* Drops cached prepacked weights derived from the fd (call after rewriting a
 * weight tensor in place).  Returns the number of cache entries dropped. */
int htp_ops_amd_invalidate_weights(int fd);

#ifdef __cplusplus
}
#endif

#endif /* HTP_OPS_RPCMEM_H */
