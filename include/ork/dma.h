/* ork/dma.h -- host buffers the device reads/writes efficiently (MI355X build). Part of <ork_npu.h>. */
#ifndef ORK_DMA_H
#define ORK_DMA_H
/* reference include/ork/dma.h:21. Pinned, device-mapped host memory (hipHostMalloc). Pass it (or any
 * pointer inside it) as A or C: runs move it with direct DMA instead of a pageable staging copy.
 * NULL on failure, on an offline context, or when the 64-entry table is full. */
void        *ork_dma_alloc(ork_npu *ctx, size_t size);
/* reference include/ork/dma.h:27 */
void         ork_dma_free(ork_npu *ctx, void *ptr);
#endif
