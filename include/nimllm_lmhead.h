/*
 * nimllm_lmhead.h -- C ABI of the MI355X (gfx950) output projection.
 *
 * The LM head of nimllm's forward pass, on the device: the logits
 * y[b, r] = W[r, :] . x[b, :] for a GGUF weight matrix W (rows = vocabulary,
 * cols = model width) and nb normalised hidden states x, written straight to
 * HBM where nls_sample (nimllm_sampler.h) reads them.  It replaces
 *
 *   matmul(m.output, addr ctx.xb[0], addr ctx.logits[0], 1)   model.nim:470
 *   matmul(m.output, addr ctx.xb[0], addr allLogits[base], B) model.nim:466
 *
 * i.e. `matmul` (src/nimllm/model.nim:179-200, matmulTask :144-170) on the
 * output matrix, and returns the same fp32 bits:
 *   - the int8 activation path when the reference takes it (model.nim:185:
 *     exactMatmul off, actBlockLen(type) > 0, cols a multiple of it, and
 *     nb <= 4 or a type other than Q8_0): quantizeAct then dotRowAct
 *     (quant.nim:646-798) for Q4_K, Q5_K, Q6_K, Q8_0 and Q4_0;
 *   - otherwise dequantRow then dotF32 (quant.nim:336-374) for every type the
 *     reference reads: F32, F16, BF16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K,
 *     Q3_K, Q4_K, Q5_K, Q6_K, Q8_K;
 *   - plus the LoRA term y += scale * B (A x) when an adapter is attached
 *     (model.nim:189-200; applyLora attaches one to an untied output, :526).
 * Parity holds for finite weights and activations; a NaN input gives a NaN
 * wherever the reference gives one, with a payload that may differ.
 *
 * Status codes are nimllm_sampler.h's NLS_* values.  Nothing here allocates:
 * the caller passes a device workspace of nls_lm_head_workspace() bytes.
 */
#ifndef NIMLLM_LMHEAD_H
#define NIMLLM_LMHEAD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type codes (quant.nim:14-19) accepted as `ggml_type`. */
enum {
  NLS_GGML_F32 = 0, NLS_GGML_F16 = 1, NLS_GGML_Q4_0 = 2, NLS_GGML_Q4_1 = 3,
  NLS_GGML_Q5_0 = 6, NLS_GGML_Q5_1 = 7, NLS_GGML_Q8_0 = 8, NLS_GGML_Q2_K = 10,
  NLS_GGML_Q3_K = 11, NLS_GGML_Q4_K = 12, NLS_GGML_Q5_K = 13, NLS_GGML_Q6_K = 14,
  NLS_GGML_Q8_K = 15, NLS_GGML_BF16 = 30
};

/* A LoRA adapter on the output matrix (LoraPair, model.nim:34-39): a is
 * [rank, cols] and b is [rows, rank], row-major fp32 on the device. */
typedef struct nls_lora {
  const float* d_a;
  const float* d_b;
  int32_t rank;
  float scale;
} nls_lora;

/* rowBytes(type, cols) (quant.nim:65-70): the bytes of one weight row, or -1
 * for a type the reference cannot read or a cols that is not whole blocks
 * (where rowBytes raises).  d_weight must hold rows times this. */
int64_t nls_lm_head_row_bytes(int32_t ggml_type, int64_t cols);

/* Bytes of device workspace nls_lm_head needs for these sizes (0 when the
 * call needs none).  `exact` is the reference's exactMatmul switch
 * (model.nim:173-175).  Returns 0 for an unsupported type as well. */
size_t nls_lm_head_workspace(int32_t ggml_type, int64_t cols, int32_t nb, int32_t lora_rank,
                             int32_t exact);

/*
 * y[nb, rows] = x[nb, cols] . W^T (+ LoRA), as matmul(w, x, y, nb) does
 * (model.nim:179-200).  d_weight holds `rows` rows of rowBytes(type, cols)
 * bytes each (the GGUF tensor data, quant.nim:65-70), 16-byte aligned; d_x is
 * [nb, cols] fp32, 16-byte aligned; d_y is [nb, rows] fp32.  `lora` may be
 * NULL.  d_work is a device buffer of at least nls_lm_head_workspace() bytes,
 * 256-byte aligned (any pointer when that size is 0).  Stream-ordered on
 * `stream` (a hipStream_t, NULL = default stream); does not synchronise.
 * Errors: NLS_ERR_INVALID_ARGUMENT for a type the reference cannot read, a
 * cols that is not a multiple of the type's block (rowBytes raises there),
 * NULL or misaligned pointers, or a short workspace; NLS_ERR_UNSUPPORTED
 * when cols exceeds what one workgroup's LDS holds on the int8 path
 * (more than 1024 blocks per row); nb == 0 or rows == 0 does nothing.
 */
int32_t nls_lm_head(const void* d_weight, int32_t ggml_type, int64_t rows, int64_t cols,
                    const float* d_x, int32_t nb, float* d_y, int32_t exact, const nls_lora* lora,
                    void* d_work, size_t work_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif
