/*
 * shs_oracle.h — CPU restatement of llm-shield's Shieldstral prefill arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the HIP path is compared
 * against, and the timed CPU baseline ("port") in bench.py. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it; the product
 * library (libshieldstral_hip) never links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to the
 * llm-shield repository). Pinning status of each function is listed in the
 * header comment of shs_oracle.c.
 */
#ifndef SHS_ORACLE_H
#define SHS_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (ggml.h numbering, GgmlType.cs:10-44). */
enum {
    ORA_F32 = 0, ORA_F16 = 1, ORA_Q4_0 = 2, ORA_Q4_1 = 3,
    ORA_Q5_0 = 6, ORA_Q5_1 = 7, ORA_Q8_0 = 8
};

/* ------------------------------------------------------------- fp16 */
float    ora_half_to_float(uint16_t h);
uint16_t ora_float_to_half(float f);            /* round to nearest even */

/* ------------------------------------------------- block geometry / decode */
int     ora_type_size(int type);                /* bytes per 32-block */
int64_t ora_row_bytes(int type, int64_t cols);
int     ora_dequantize(int type, const uint8_t* src, float* dst, int64_t n);
/* ggml/gguf-py weight quantizer (offline, synthetic weights). */
int     ora_quantize(int type, const float* src, uint8_t* dst, int64_t n);

/* ------------------------------------------------ activation quantization */
/* IntegerGemm.QuantizeActivations: fp32 scale, ties-to-even (IntegerGemm.cs:97-138). */
void ora_quantize_activations(const float* x, int64_t n, int8_t* q, float* d, int32_t* s);
/* IntegerDot.QuantizeActivations: fp16 stored scale, half away from zero, clamp ±127
 * (IntegerDot.cs:60-98). d receives the fp16-rounded scale as fp32. */
void ora_quantize_activations_q8(const float* x, int64_t n, int8_t* q, float* d, int32_t* s);

/* ------------------------------------------------------------------ GEMM */
/* Integer block sums I[t][r][b] = Σ_k (u−z)·q (IntegerGemm.cs:371-419). */
int ora_block_sums(int type, const uint8_t* w, int rows, int cols,
                   const int8_t* q, const int32_t* s, int tokens, int32_t* out);
/* y[t][r] for already-quantized activations, rows = row_ids (or all when NULL). */
int ora_matmul_q(int type, const uint8_t* w, int rows, int cols,
                 const int8_t* q, const float* d, const int32_t* s, int tokens,
                 const int32_t* row_ids, int n_ids, float* y, int threads);
/* QuantMatMul.ForwardAsync / ForwardRowsAsync (QuantMatMul.cs:71-110,292-410):
 * quantize x once, then the per-block epilogue. semantics: 0 IntegerGemm, 1 IntegerDot. */
int ora_matmul(int type, const uint8_t* w, int rows, int cols, const float* x, int tokens,
               const int32_t* row_ids, int n_ids, float* y, int semantics, int threads);
/* QuantMatMul.GatherRows (QuantMatMul.cs:534-545). */
int ora_gather_rows(int type, const uint8_t* table, int rows, int cols,
                    const int32_t* ids, int n, float* out);

/* ------------------------------------------------------------ elementwise */
void ora_rmsnorm(const float* x, const float* w, float eps, int n, float* y);      /* Kernels.cs:26-61 */
float ora_expf(float x);                                                          /* TensorPrimitives.Exp */
void ora_expf_n(const float* x, int64_t n, float* y);
void ora_swiglu(const float* gate, float* up, float* dst, int64_t n);              /* Kernels.cs:83-90 */
void ora_softmax(float* x, int n);                                                 /* Kernels.cs:103-122 */
void ora_dot4(const float* shared, const float* a0, const float* a1, const float* a2,
              const float* a3, int n, float* r);                                   /* Kernels.cs:157-186 */
void ora_add_scaled4(const float* src, float* d0, float* d1, float* d2, float* d3,
                     const float w[4], int n);                                     /* Kernels.cs:193-220 */

/* --------------------------------------------------------------- model */
typedef struct {
    int   n_layer, hidden, n_head, n_kv_head, head_dim, ffn, vocab;
    float eps;
    float rope_theta;        /* freq_base */
    int   rope_dim;
    float rope_scale;        /* YaRN factor; 1 = off */
    int   rope_orig_ctx;
    float yarn_beta_fast, yarn_beta_slow, yarn_ext_factor;
    float yarn_mscale, yarn_mscale_all_dim, rope_attn_factor;
    float attn_temperature;  /* Llama-4 beta; 0 = off */
    int   yarn_active;       /* ModelConfig.YarnActive */
} ora_config;

typedef struct {
    int type_q, type_k, type_v, type_o, type_gate, type_up, type_down;
    const uint8_t *q, *k, *v, *o, *gate, *up, *down;
    const float *attn_norm, *ffn_norm;
} ora_layer;

typedef struct {
    ora_config cfg;
    int embd_type;
    const uint8_t* token_embd;   /* [vocab][hidden], tied head */
    const float* output_norm;
    const ora_layer* layers;
} ora_model;

/* KvCache (KvCache.cs:12-139): per layer [head][cap][dim], fp32. */
typedef struct {
    float* k;   /* n_layer * n_kv_head * cap * head_dim */
    float* v;
    int cap, len;
} ora_kv;

/* Rope ctor (Rope.cs:33-66): freqs[rope_dim/2] and the magnitude scale. */
void ora_rope_freqs(const ora_config* cfg, float* freqs, float* mscale);
/* Rope.Apply (Rope.cs:112-135) for one token, heads × head_dim contiguous. */
void ora_rope_apply(const float* freqs, float mscale, int rope_dim,
                    float* data, int heads, int head_dim, int position);

typedef void (*ora_capture_fn)(const char* name, const float* data, int rows, int cols, void* user);

/* MinistralModel.ForwardAsync (MinistralModel.cs:183-271).
 * head_mode 0: prefill only; 1: selected vocab rows; 2: full vocabulary.
 * Appends at kv->len (caller provides capacity ≥ len + n). */
int ora_forward(const ora_model* m, ora_kv* kv, const int32_t* tokens, int n,
                int head_mode, const int32_t* vocab_ids, int n_ids, float* logits,
                ora_capture_fn capture, void* user, int threads);

/* One decoder layer (MinistralModel.cs:216-237) on hidden state x[n][hidden] at
 * positions 0..n-1 of the cache, y receives the layer output. */
int ora_layer_forward(const ora_model* m, ora_kv* kv, int layer, const float* x, int n, float* y, int threads);

/* ShieldstralModerator.Score (ShieldstralModerator.cs:348-364). */
void ora_score(const float* logits, int n_yes, int n_no, float* score, float* yes, float* no);

#ifdef __cplusplus
}
#endif
#endif
