/*
 * moe_safetensors.h — C ABI of the checkpoint reader in libmoehip.so: the
 * safetensors bundle FFAI loads its weights from, and the stacked
 * mlx-affine expert triplets that feed the grouped kernels of moe_hip.h
 * without repacking.
 *
 * Reference interfaces (paths relative to the FFAI checkout):
 *   SafeTensorsFile / SafeTensorsBundle  Sources/FFAI/Loader/SafeTensors.swift
 *   QuantizedTriplet / isQuantized       SafeTensors.swift:377-396
 *   deriveAffineQuantBits                Sources/FFAI/Layers.swift:348-363
 *   stacked expert load                  Models/Text/Qwen3xText.swift:682-800,
 *                                        Models/Text/Gemma4Text.swift:540-555
 *
 * Conventions
 *  - A bundle keeps every file memory-mapped read-only until moe_st_close;
 *    tensor bytes are copied out on request (to host memory, or to device
 *    memory through pinned staging buffers). The reference copies every
 *    tensor at open and unmaps at once (SafeTensors.swift:88-99); here
 *    nothing is copied until a tensor is asked for, so a caller can stream
 *    one layer's experts at a time into HBM.
 *  - Errors return a moe_status with moe_last_error_string() naming the
 *    cause in the reference's words (file not found, header smaller than
 *    8 bytes, JSON header malformed, malformed entry for tensor "x",
 *    tensor "x" not present).
 *  - Tensors of dtypes outside moe_st_dtype are skipped at open, as the
 *    reference does (SafeTensors.swift:170-185): looking one up reports a
 *    missing tensor.
 *  - A bundle is not reentrant; use one per thread.
 */
#ifndef MOE_SAFETENSORS_H
#define MOE_SAFETENSORS_H

#include <stddef.h>
#include <stdint.h>

#include "moe_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* DType.fromSafeTensors (Sources/FFAI/DType.swift:42-55); the first three
 * share moe_dtype's numbering. */
typedef enum moe_st_dtype {
    MOE_ST_F32 = 0,
    MOE_ST_F16 = 1,
    MOE_ST_BF16 = 2,
    MOE_ST_I32 = 3,
    MOE_ST_U32 = 4,
    MOE_ST_I64 = 5,
    MOE_ST_U64 = 6,
    MOE_ST_I8 = 7,
    MOE_ST_U8 = 8
} moe_st_dtype;

#define MOE_ST_MAX_DIMS 8

typedef struct moe_st_bundle* moe_st_t;

/* SafeTensorsBundle.init(directory:) (SafeTensors.swift:248-292) when path
 * is a directory: model.safetensors.index.json's weight_map files, else
 * model.safetensors, else every *.safetensors in name order; or
 * SafeTensorsFile.init(url:) (SafeTensors.swift:101-230) when path is a
 * file. Symlinks are resolved (Hugging Face cache snapshots). */
moe_status moe_st_open(const char* path, moe_st_t* out);
void moe_st_close(moe_st_t bundle);

/* SafeTensorsBundle.allKeys (SafeTensors.swift:363): count and the i-th
 * name in sorted order. The string lives as long as the bundle. */
int64_t moe_st_count(moe_st_t bundle);
const char* moe_st_name(moe_st_t bundle, int64_t i);

/* Entry metadata (SafeTensorsFile.Entry, SafeTensors.swift:70-76). shape
 * receives ndim entries (ndim <= MOE_ST_MAX_DIMS); nbytes the byte size. */
moe_status moe_st_info(moe_st_t bundle, const char* name, int32_t* dtype, int32_t* ndim,
                       int64_t* shape, size_t* nbytes);

/* SafeTensorsBundle.tensor(named:) (SafeTensors.swift:294-299): the
 * tensor's bytes, bytes == nbytes exactly. moe_st_read_host copies into
 * host memory; moe_st_upload into device memory on `stream` and returns
 * once the bytes are in place (the staging buffers are reused). */
moe_status moe_st_read_host(moe_st_t bundle, const char* name, void* dst, size_t bytes);
moe_status moe_st_upload(moe_st_t bundle, const char* name, void* dst_device, size_t bytes,
                         hipStream_t stream);

/* SafeTensorsBundle.isQuantized (SafeTensors.swift:370-372): 1 when
 * <base>.weight, <base>.scales and <base>.biases are all present. */
int32_t moe_st_is_quantized(moe_st_t bundle, const char* base);

/* Device bytes moe_st_load_stacked needs for the triplet at base: weight,
 * scales and biases each 256-byte aligned. */
moe_status moe_st_stacked_bytes(moe_st_t bundle, const char* base, int32_t group_size,
                                size_t* bytes);

/* A stacked mlx-affine projection (QuantizedTriplet, SafeTensors.swift:
 * 374-396, as the stacked-expert loaders read it: Qwen3xText.swift:682-800,
 * Gemma4Text.swift:540-555): <base>.weight [E, N, K*bits/32] u32 (or a 2-D
 * [N, K*bits/32] single expert, E = 1), <base>.scales and <base>.biases
 * [E, N, K/group_size] in one f16/bf16/f32 dtype. bits comes from the
 * shapes (deriveAffineQuantBits, Layers.swift:348-363), per tensor, so
 * mixed-precision checkpoints load as they are. The three tensors are
 * uploaded into dst_device (moe_st_stacked_bytes bytes, 256-byte aligned)
 * and *out describes them for moe_hip.h (out_bias NULL). */
moe_status moe_st_load_stacked(moe_st_t bundle, const char* base, int32_t group_size,
                               void* dst_device, size_t dst_bytes, moe_qproj* out,
                               hipStream_t stream);

/* moe_st_load_stacked for `count` triplets in one pass (a layer's gate, up
 * and down stacks, say): every triplet is validated before any byte moves,
 * then all of them stream through one queue of host-to-device copies. No
 * counterpart in the reference, which loads each triplet on its own
 * (Qwen3xText.swift:700-722). */
moe_status moe_st_load_stacked_many(moe_st_t bundle, int32_t count, const char* const* bases,
                                    int32_t group_size, void* const* dst_device,
                                    const size_t* dst_bytes, moe_qproj* out, hipStream_t stream);

/* GPT-OSS MXFP4 expert stacks (transcodeStackedExperts, Models/Text/
 * GPTOSSText.swift:1071-1236): <base>.weight [E, N, K/8] u32 (fp4 codes),
 * <base>.scales [E, N, K/32] u8 (e8m0 exponents) and <base>.bias [E, N]
 * (f16, bf16 or f32; 2-D tensors are one expert). moe_st_mxfp4_bytes gives
 * the device bytes of the loaded projection and the scratch bytes the load
 * stages through; moe_st_load_mxfp4 uploads the three tensors, transcodes
 * them on the GPU to an affine 4-bit triplet with group size 32 (scales and
 * biases in act_dtype, moe_mxfp4_to_affine) and converts the per-row bias to
 * act_dtype as out_bias. *out describes the result for moe_hip.h. The
 * transcode is queued on `stream` after the copies: keep the scratch until
 * the stream has passed it. */
moe_status moe_st_mxfp4_bytes(moe_st_t bundle, const char* base, int32_t act_dtype,
                              size_t* bytes, size_t* scratch_bytes);
moe_status moe_st_load_mxfp4(moe_st_t bundle, const char* base, int32_t act_dtype,
                             void* dst_device, size_t dst_bytes, void* scratch_device,
                             size_t scratch_bytes, moe_qproj* out, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* MOE_SAFETENSORS_H */
