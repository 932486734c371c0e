/*
 * weights.h -- the weight buffers of a ggml backend on MI355X (C ABI): what the reference backend's
 * buffer type allocates for a tensor and what its set_tensor / get_tensor do
 * (integrations/llama.cpp/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp: weight_shape_ok :103-109,
 * stream_bytes :116-118, buft get_alloc_size :259-266, buffer_set_tensor :175-191,
 * buffer_get_tensor :193-206).
 *
 * A K-quant weight (KC_QTYPE_Q4_K / KC_QTYPE_Q6_K, rows % 8 == 0, k % 256 == 0) lives on the
 * device as the repacked stream the matvec and matmul kernels read (kcKquantStreamBytes bytes,
 * not ggml's); it is uploaded whole (set: the ggml blocks, offset 0 and every byte -- the
 * reference asserts the same) and read back as ggml blocks, any byte range of them (unpack).
 * Every other tensor (f32, and fp16 weights, which the kernels read in ggml's row-major layout)
 * is a plain copy of the byte range. The copies go to the given stream and the calls return once
 * they are done (the host buffer may be reused); each K-quant call stages the ggml bytes in a
 * device buffer of their size.
 */
#ifndef KERNELCORE_WEIGHTS_H
#define KERNELCORE_WEIGHTS_H

#include "kc.h"

/* Bytes to allocate on the device for a rows x k tensor of qtype (KC_QTYPE_F32 0, KC_QTYPE_F16 1,
 * KC_QTYPE_Q4_K 12, KC_QTYPE_Q6_K 14): the stream for a K-quant weight, ggml's size otherwise. */
KC_API kcError_t kcWeightAllocSize(int qtype, int rows, int k, size_t* bytes) KC_NOEXCEPT;
/* set_tensor: host bytes [offset, offset + size) of the tensor's ggml form into dst. */
KC_API kcError_t kcWeightSetTensor(int qtype, int rows, int k, void* dst, const void* host, size_t offset,
                                   size_t size, kcStream_t stream KC_DEF(nullptr)) KC_NOEXCEPT;
/* get_tensor: bytes [offset, offset + size) of the tensor's ggml form, read from src, into host. */
KC_API kcError_t kcWeightGetTensor(int qtype, int rows, int k, const void* src, void* host, size_t offset,
                                   size_t size, kcStream_t stream KC_DEF(nullptr)) KC_NOEXCEPT;
/* memset_tensor: bytes [offset, offset + size) of the tensor's ggml form set to value (its low
 * byte), so that a later get_tensor reads value there (buffer_memset_tensor,
 * ggml-kernelcore.cpp:171-173, which sets the repacked memory itself). A K-quant weight is
 * unpacked, set and repacked on the device (its stream holds exactly the ggml bytes, rearranged);
 * any other tensor is a plain device memset of the range. */
KC_API kcError_t kcWeightMemsetTensor(int qtype, int rows, int k, void* dst, int value, size_t offset, size_t size,
                                      kcStream_t stream KC_DEF(nullptr)) KC_NOEXCEPT;

#endif /* KERNELCORE_WEIGHTS_H */
