/* titan_ckpt.h -- checkpoint reading and load-time repack to the gfx950
 * TILED layout (host code; no GPU calls).
 *
 * Replaces the reference's weight readers, which copy raw bytes to the GPU
 * and never repack:
 *   safetensors   ModelLoader::load / load_single / load_sharded and
 *                 read_tensor_cpu (src/model/loader.cpp:140-472, header parse
 *                 :36-138)
 *   GGUF          GGUFLoader::load / read_tensor_cpu
 *                 (src/model/gguf_loader.cpp:60-240, 299-320; types
 *                 src/model/gguf_loader.h:29-100)
 *   NVFP4 experts MoEExecutor::load_nvfp4_expert (src/model/moe.cpp:613-724):
 *                 <base>.weight (U8), <base>.weight_scale (F8_E4M3),
 *                 <base>.weight_scale_2 (F32 or BF16 scalar, 1.0 if absent)
 *   titan-v1      the packed INT4 blobs written by tools/convert_titan.py:158-198
 *                 (manifest.json + *.bin; weights | fp16 scales | fp16 biases)
 *
 * titan_ckpt_open accepts a .safetensors file, a .gguf file, or a directory
 * holding model.safetensors.index.json (+ shards), model.safetensors, other
 * *.safetensors files, or a titan-v1 manifest.json.  All functions return a
 * TITAN_* status from titan_qmm.h (0 = ok).
 */
#ifndef TITAN_CKPT_H
#define TITAN_CKPT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct titan_ckpt titan_ckpt;

/* element types of stored tensors */
enum {
    TITAN_CK_F32 = 0,
    TITAN_CK_F16 = 1,
    TITAN_CK_BF16 = 2,
    TITAN_CK_F64 = 3,
    TITAN_CK_I8 = 4,
    TITAN_CK_U8 = 5,
    TITAN_CK_I16 = 6,
    TITAN_CK_I32 = 7,
    TITAN_CK_I64 = 8,
    TITAN_CK_BOOL = 9,
    TITAN_CK_F8_E4M3 = 10,
    TITAN_CK_F8_E5M2 = 11,
    TITAN_CK_GGML = 100,      /* GGUF block-quantized: see ggml_type */
    TITAN_CK_INT4_AFFINE = 200 /* titan-v1 int4: codes | fp16 scales | fp16 biases */
};

typedef struct {
    const char* name;  /* owned by the checkpoint */
    int dtype;         /* TITAN_CK_* */
    int ggml_type;     /* GGUF type id (gguf_loader.h:29-61), -1 otherwise */
    int ndim;
    int64_t shape[8];  /* outermost first (GGUF dims are reversed to match) */
    uint64_t nbytes;   /* bytes stored in the file */
    int group_size;    /* titan-v1 int4 only */
} titan_ckpt_tensor;

/* A quantized weight as the GEMV / GEMM entry points take it. */
typedef struct {
    int format;         /* TITAN_INT4 / TITAN_NVFP4 / TITAN_Q4_K / TITAN_Q3_K */
    int rows, cols, group_size;
    float global_scale; /* NVFP4 weight_scale_2, else 1 */
    size_t tiled_bytes; /* size of the TILED buffer */
} titan_ckpt_weight;

int titan_ckpt_open(const char* path, titan_ckpt** out);
void titan_ckpt_close(titan_ckpt* ck);
int titan_ckpt_count(const titan_ckpt* ck);
int titan_ckpt_tensor_at(const titan_ckpt* ck, int index, titan_ckpt_tensor* out);
/* index of a tensor by name, or -1 */
int titan_ckpt_find(const titan_ckpt* ck, const char* name);
/* raw stored bytes of tensor `index` (dst_bytes >= nbytes) */
int titan_ckpt_read(const titan_ckpt* ck, int index, void* dst, size_t dst_bytes);

/* `name` is a GGUF Q4_K / Q3_K tensor, a titan-v1 int4 tensor, or the base
 * name of an NVFP4 projection (e.g. "model.layers.0.mlp.experts.3.gate_proj").
 * weight_info describes what load_tiled produces; load_tiled reads the parts
 * and writes the TILED layout (titan_repack_host) into host memory. */
int titan_ckpt_weight_info(const titan_ckpt* ck, const char* name, titan_ckpt_weight* out);
int titan_ckpt_load_tiled(const titan_ckpt* ck, const char* name, void* tiled, size_t tiled_bytes,
                          titan_ckpt_weight* out);

#ifdef __cplusplus
}
#endif
#endif /* TITAN_CKPT_H */
