/*
 * mi_ckpt.h -- C ABI of the quantized-checkpoint loader that feeds mi_qmm.h.
 *
 * Reads an MLX model directory (config.json + *.safetensors) into host-visible
 * tensor records and copies them into the caller's buffers, so the packed
 * weights, scales and biases land exactly where mi_quantized_matmul and
 * mi_gather_qmm read them. Replaces, for this path:
 *   - the "quantization" block of parseConfig         src/model.zig:1480-1505
 *   - loadWeights / loadWeightsSingleFile / loadSafetensorsFile (which call
 *     mlx_load_safetensors, src/mlx.zig:170)         src/model.zig:2946-3146
 *   - the weight-name binding of a quantized linear:
 *     getLayerWeight / getLayerScaleOrEmpty / getLayerBias
 *                                                     src/transformer.zig:21068-21153
 *   - per-weight (bits, group_size, mode) resolution: computeQuantParams
 *                                                     src/transformer.zig:16876-16924
 *
 * Files are memory-mapped read-only; nothing is copied until mi_ckpt_read or
 * mi_ckpt_upload. Return codes are mi_qmm.h's (MI_OK, MI_ERR_INVALID for a
 * malformed file, missing tensor or unsupported declaration, MI_ERR_HIP for a
 * failed device copy); mi_last_error() holds the message.
 */
#ifndef MI_CKPT_H
#define MI_CKPT_H
#include <stddef.h>
#include <stdint.h>

#include "mi_qmm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* QuantMode (src/model.zig:19-43). */
enum { MI_QMODE_AFFINE = 0, MI_QMODE_NVFP4 = 1, MI_QMODE_MXFP4 = 2, MI_QMODE_MXFP8 = 3 };

typedef struct mi_ckpt mi_ckpt;

/* Model-wide quantization declared by config.json's top-level "quantization"
 * object (src/model.zig:152-156, 1480-1505). bits == 0: dense checkpoint (no
 * such key); group_size then keeps its default 64, mode affine. */
typedef struct {
  int bits;
  int group_size;
  int mode;
} mi_quant_config;

#define MI_CKPT_MAX_DIMS 8

/* One tensor as the loader hands it out. dtype is an mlx_dtype code
 * (src/mlx.zig:20-35). A float16 tensor named *.scales / *.biases, or any 1-D
 * float16 tensor, reports bfloat16: it is narrowed on read, as
 * narrowsLoadedF16 (src/model.zig:3057-3061) does at load. nbytes is the size
 * after that narrowing. */
typedef struct {
  int dtype;
  int ndim;
  int64_t shape[MI_CKPT_MAX_DIMS];
  int64_t nbytes;
} mi_tensor_info;

/* The tensors of one quantized linear layer "{prefix}.weight/.scales/.biases"
 * and the (bits, group_size, mode) the matmul must be called with.
 *   has_scales  0 for a dense checkpoint (quant_bits == 0): weight is plain.
 *   has_biases  affine: always 1 (a missing .biases is an error); fp modes: 1
 *               only when the checkpoint carries an affine override's biases.
 *   in_dim      input dimension (K) the parameters were solved for. */
typedef struct {
  int has_scales;
  int has_biases;
  int bits;
  int group_size;
  int mode;
  int64_t out_dim;
  int64_t in_dim;
} mi_linear_desc;

/* Open an MLX model directory: config.json (optional: absent means dense) and
 * every *.safetensors in it, in name order; a key found in two files keeps the
 * later file's tensor. load_vision=0 drops the vision/audio tower keys as
 * shouldKeepWeightKey (src/model.zig:3148-3185). A directory with no usable
 * tensor is an error (the reference's error.NoWeightFiles). */
int mi_ckpt_open(const char* model_dir, int load_vision, mi_ckpt** out);

/* Open one .safetensors file (loadWeightsSingleFile, src/model.zig:2953-2969);
 * no config.json is read, so the quantization is dense until
 * mi_ckpt_set_quant_config names one. */
int mi_ckpt_open_file(const char* path, mi_ckpt** out);

void mi_ckpt_close(mi_ckpt* ck);

/* Parse only the "quantization" block of a config.json text (no files touched). */
int mi_parse_quant_config(const char* json, size_t len, mi_quant_config* out);

int mi_ckpt_quant_config(const mi_ckpt* ck, mi_quant_config* out);
int mi_ckpt_set_quant_config(mi_ckpt* ck, const mi_quant_config* cfg);

/* Number of tensors, and the i-th name in sorted order (pointer valid until close). */
int64_t mi_ckpt_count(const mi_ckpt* ck);
const char* mi_ckpt_name(const mi_ckpt* ck, int64_t i);

/* MI_OK, or MI_ERR_INVALID when the tensor does not exist. */
int mi_ckpt_info(const mi_ckpt* ck, const char* name, mi_tensor_info* info);

/* Copy a tensor's bytes (narrowed as mi_ckpt_info reports) into host memory
 * dst of at least `bytes` (= info.nbytes). */
int mi_ckpt_read(const mi_ckpt* ck, const char* name, void* dst, size_t bytes);

/* Same into DEVICE memory dst; synchronous (the copy is complete on return). */
int mi_ckpt_upload(const mi_ckpt* ck, const char* name, void* dst, size_t bytes);

/* Bind "{prefix}.weight/.scales/.biases" and resolve the layer's parameters
 * against the model-wide declaration and the weight's packed geometry:
 * uint8 scales are an fp mode, float scales affine; in_dim > 0 solves the exact
 * per-weight (bits, group_size) the way computeQuantParams does when the caller
 * knows the activation's inner dimension; in_dim == 0 takes it from the
 * declaration. MI_ERR_INVALID names the first missing tensor. */
int mi_ckpt_linear(const mi_ckpt* ck, const char* prefix, int64_t in_dim, mi_linear_desc* out);

#ifdef __cplusplus
}
#endif
#endif
