/*
 * nls_oracle_quant.h -- CPU restatement of nimllm's output projection
 * (the LM head): the quantised-weight formats, the int8 activation path and
 * the float32 dot product that `matmul` (src/nimllm/model.nim:144-200) runs
 * for `m.output` (model.nim:461-470).
 *
 * TEST INFRASTRUCTURE ONLY, like the sampler restatement in nls_oracle.h:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it; the product path never links or calls it.
 *
 * Statement by statement it follows src/nimllm/quant.nim:
 *   halfToFloatSlow :83-98, bf16ToFloat :138, getScaleMinK4 :156-162,
 *   dequantBlock :164-334, dequantRow :336-352, dotF32 :362-374,
 *   actBlockLen :639-644, quantizeAct :646-667, dotQ4K :669-695,
 *   dotQ5K :697-729, dotQ6K :731-760, dotQ8_0i :762-772, dotQ4_0i :774-786,
 *   dotRowAct :788-798
 * and src/nimllm/model.nim: matmulTask :144-170, matmul :179-200 (including
 * the LoRA term :189-200 and the `exactMatmul` switch :173-175).
 * fp32 arithmetic runs in the reference's order; the file is compiled with
 * -O2 -ffp-contract=off (no FMA, no fast-math), as the reference's own test
 * build is (tests/config.nims:1-3).
 */
#ifndef NLS_ORACLE_QUANT_H
#define NLS_ORACLE_QUANT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type codes (quant.nim:14-19). */
enum {
  NLO_F32 = 0, NLO_F16 = 1, NLO_Q4_0 = 2, NLO_Q4_1 = 3, NLO_Q5_0 = 6, NLO_Q5_1 = 7,
  NLO_Q8_0 = 8, NLO_Q2_K = 10, NLO_Q3_K = 11, NLO_Q4_K = 12, NLO_Q5_K = 13,
  NLO_Q6_K = 14, NLO_Q8_K = 15, NLO_BF16 = 30
};

/* Elements per block and bytes per block (quant.nim:38-63); 0 for a type the
 * reference cannot dequantise (supportedTypes, quant.nim:26-27). */
int32_t nlo_block_size(int32_t type);
int32_t nlo_type_size(int32_t type);
/* rowBytes (quant.nim:65-70): -1 when n is not a multiple of the block. */
int64_t nlo_row_bytes(int32_t type, int64_t n);

float nlo_half_to_float(uint16_t h);

/* dequantRow (quant.nim:336-352). Returns 0, or -1 for an unsupported type. */
int32_t nlo_dequant_row(int32_t type, const void* src, float* dst, int64_t n);

/* dotF32 (quant.nim:362-374): eight strided fp32 accumulators. */
float nlo_dot_f32(const float* a, const float* b, int64_t n);

/* actBlockLen (quant.nim:639-644). */
int32_t nlo_act_block_len(int32_t type);

/* quantizeAct (quant.nim:646-667) of n floats in blocks of block_len:
 * d[n / block_len], qs[n], and for block_len 256 bsums[n / 16]. */
void nlo_quantize_act(const float* x, int64_t n, int32_t block_len, float* d, int8_t* qs,
                      int32_t* bsums);

/* dotRowAct (quant.nim:788-798) against the activation elements
 * off .. off + n - 1 (off and n multiples of the block). */
float nlo_dot_row_act(int32_t type, const void* row, const float* act_d, const int8_t* act_qs,
                      const int32_t* act_bsums, int64_t off, int64_t n);

/* 1 when matmul quantises the activations (model.nim:185). */
int32_t nlo_matmul_uses_act(int32_t type, int64_t cols, int32_t nb, int32_t exact);

/* matmul (model.nim:179-200): y[nb, rows] = x[nb, cols] . W^T, W stored as
 * `rows` rows of rowBytes(type, cols) bytes.  `exact` is `exactMatmul`
 * (model.nim:173).  lora_a [rank, cols] and lora_b [rows, rank] may be NULL
 * (rank 0).  Rows first .. last - 1 only (last = rows for all of them), so a
 * sample of rows can be timed; the other entries of y are left alone.
 * Returns 0, or -1 for an unsupported type or a cols that is not a multiple
 * of the block. */
int32_t nlo_matmul(int32_t type, const void* w, int64_t rows, int64_t cols, const float* x,
                   int32_t nb, float* y, int32_t exact, const float* lora_a,
                   const float* lora_b, int32_t lora_rank, float lora_scale, int64_t first,
                   int64_t last);

#ifdef __cplusplus
}
#endif

#endif
