/*
 * miqmm_checkpoint.h -- C ABI for reading MLX's on-disk quantized checkpoints
 * (host only: no GPU call).
 *
 * A model directory holds config.json and either model.safetensors or
 * model.safetensors.index.json naming several shards
 * (src/engine/mlx_native.rs:3603-3623).  A module is stored quantized iff a
 * "<path>.scales" tensor exists; its bits and group size come from
 * config.json's "quantization" (or "quantization_config") object, whose
 * per-module objects override the top-level default
 * (src/engine/mlx_lm/models/gemma4.rs:1755-1834,
 * src/engine/mlx_lm/models/qwen3_5.rs:722-760).  The codes are
 * "<path>.weight", which mlx-rs names "<path>.inner.weight"
 * (src/engine/mlx_native.rs:3684-3703); both are accepted.  Each module's bits
 * and group size are checked against its tensor shapes; a mismatch fails
 * the open with MIQMM_EINVAL instead of loading misread words (shapes fix
 * only the product bits * group_size, so a misdescription keeping it passes).
 *
 * Replaces the reference's per-model load functions (e.g. load_llama_any,
 * src/engine/mlx_native.rs:3585-3760) for the quantized modules: the caller
 * gets, per module, the tensors to hand to miqmm_quantized_matmul /
 * miqmm_quantized_embedding / miqmm_gather_qmm and reads their bytes with
 * miqmm_checkpoint_read (then copies them to the device).  Status codes are
 * those of miqmm.h; messages via miqmm_checkpoint_last_error().
 */
#ifndef MIQMM_CHECKPOINT_H
#define MIQMM_CHECKPOINT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct miqmm_checkpoint miqmm_checkpoint;

/* One quantized module.  Strings are owned by the checkpoint handle. */
typedef struct miqmm_qmodule {
    const char* path;    /* e.g. "model.layers.0.self_attn.q_proj" */
    const char* weight;  /* tensor names: packed codes (U32) */
    const char* scales;
    const char* biases;
    const char* bias;    /* the Linear's bias, or NULL */
    int bits, group_size;
    int sb_dtype;        /* MIQMM_DT_BF16 or MIQMM_DT_F16 */
    int64_t experts;     /* 0: codes [rows, cols*bits/32]; E: stacked [E, rows, cols*bits/32] */
    int64_t rows, cols;  /* N and K of each matrix */
} miqmm_qmodule;

typedef struct miqmm_tensor_info {
    const char* name;
    const char* dtype;   /* safetensors dtype string: "U32", "BF16", "F16", "F32", ... */
    const char* file;    /* shard path */
    int ndim;
    int64_t shape[8];
    int64_t offset;      /* byte offset of the data in `file` */
    int64_t nbytes;
} miqmm_tensor_info;

/* Parse config.json and every shard header; build the quantization plan. */
int miqmm_checkpoint_open(const char* model_dir, miqmm_checkpoint** out);
void miqmm_checkpoint_close(miqmm_checkpoint* ckpt);

int64_t miqmm_checkpoint_num_modules(const miqmm_checkpoint* ckpt);
int64_t miqmm_checkpoint_num_tensors(const miqmm_checkpoint* ckpt);
int miqmm_checkpoint_module(const miqmm_checkpoint* ckpt, int64_t index, miqmm_qmodule* out);

/* A tensor by name, or (name == NULL) by index in [0, num_tensors). */
int miqmm_checkpoint_tensor(const miqmm_checkpoint* ckpt, const char* name, int64_t index, miqmm_tensor_info* out);

/* Copy a tensor's bytes (exactly nbytes) into host memory at dst. */
int miqmm_checkpoint_read(const miqmm_checkpoint* ckpt, const char* name, void* dst, int64_t bytes);

/* Message for the last failing checkpoint call on this thread ("" if none). */
const char* miqmm_checkpoint_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* MIQMM_CHECKPOINT_H */
