/*
 * shieldstral_hip.h — C ABI of libshieldstral_hip, the MI355X (gfx950) prefill path
 * for the Shieldstral-3B classifier behind llm-shield's ShieldstralModerator.
 *
 * The library replaces the arithmetic below ShieldstralModerator (MinistralModel,
 * QuantMatMul, IntegerGemm, Kernels, Rope, KvCache) with hand-written HIP kernels.
 * Every entry point takes plain pointers and sizes; the caller owns host buffers,
 * the library owns device memory and handles. Paths cited are in the llm-shield
 * repository (src/LlmShield.Shieldstral/...).
 *
 * Threading: a model handle owns one KV cache and one HIP stream and is not
 * thread-safe (MinistralModel.cs:21-22, ShieldstralModerator.cs:46); calls on one
 * handle must be serialised. Separate handles may be used concurrently.
 */
#ifndef SHIELDSTRAL_HIP_H
#define SHIELDSTRAL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes; the host maps them onto the reference's exception types. */
typedef enum {
    SHS_OK = 0,
    SHS_E_INVALID_ARGUMENT = 1, /* ArgumentException */
    SHS_E_OUT_OF_RANGE = 2,     /* ArgumentOutOfRangeException (QuantMatMul.cs:106-108,540-542) */
    SHS_E_INVALID_DATA = 3,     /* InvalidDataException (MinistralModel.cs:110-123) */
    SHS_E_KEY_NOT_FOUND = 4,    /* KeyNotFoundException (missing tensor) */
    SHS_E_NOT_SUPPORTED = 5,    /* NotSupportedException (IntegerGemm.cs:163) */
    SHS_E_IO = 6,               /* IOException (GgufFile.cs:156-172) */
    SHS_E_CANCELLED = 7,        /* OperationCanceledException */
    SHS_E_DEVICE = 8            /* HIP runtime failure, out of device memory, no gfx950 */
} shs_status;

/* GGML block types this library multiplies in integers (IntegerGemm.cs:58-65). */
enum { SHS_F32 = 0, SHS_F16 = 1, SHS_Q4_0 = 2, SHS_Q4_1 = 3, SHS_Q5_0 = 6, SHS_Q5_1 = 7, SHS_Q8_0 = 8 };

/* Hyperparameters, as ModelConfig holds them (ModelConfig.cs:12-60). */
typedef struct {
    int32_t n_layer, hidden, n_head, n_kv_head, head_dim, ffn, vocab;
    float   rms_eps;
    float   rope_theta;       /* rope.freq_base */
    int32_t rope_dim;
    float   rope_scale;       /* YaRN factor, 1 = none */
    int32_t rope_orig_ctx;
    float   yarn_beta_fast, yarn_beta_slow, yarn_ext_factor;
    float   yarn_mscale, yarn_mscale_all_dim, rope_attn_factor;
    float   attn_temperature; /* Llama-4 attention temperature beta, 0 = off */
    int32_t yarn_active;      /* ModelConfig.YarnActive (ModelConfig.cs:54-56) */
    char    architecture[32]; /* ModelConfig.Architecture (ModelConfig.cs:14,77): general.architecture,
                                 NUL-terminated; empty on input means "mistral3" */
} shs_config;

/* One named tensor in its native GGUF block layout, shape [ne0 = in, ne1 = out]
 * (WeightMatrix.cs:16-66). Names follow MinistralModel.cs:74-96. */
typedef struct {
    const char* name;
    int32_t     type;
    int64_t     ne0, ne1;
    const void* data;
} shs_tensor;

typedef struct shs_model shs_model;
typedef struct shs_matrix shs_matrix;

/* Thread-local description of the last failure on this thread; names the file or
 * argument and the remedy where there is one. */
const char* shs_last_error(void);

/* ------------------------------------------------------------------ model */

/* MinistralModel(GgufFile) + ShieldstralModerator.OpenAsync's load step
 * (MinistralModel.cs:59-108): validates shapes, uploads every tensor once into HBM
 * in a repacked block layout, allocates a KV cache of initial_capacity positions.
 * The caller's buffers may be released when this returns. */
shs_status shs_open_tensors(const shs_config* cfg, const shs_tensor* tensors, int32_t n_tensors,
                            int32_t device, int32_t initial_capacity, shs_model** out);

/* MinistralModel(string ggufPath) (MinistralModel.cs:56-57): memory-maps a GGUF v3
 * file (GgufFile.cs:76-199), reads ModelConfig (ModelConfig.cs:62-112) and calls
 * shs_open_tensors. The mapping is released before returning. */
shs_status shs_open(const char* gguf_path, int32_t device, int32_t initial_capacity, shs_model** out);

/* ModelConfig.FromGguf (ModelConfig.cs:62-112) on a GGUF file's header, after GgufFile's
 * header parse and truncation check (GgufFile.cs:110-172); touches no device. */
shs_status shs_read_config(const char* gguf_path, shs_config* out);

/* A random-init model of cfg's shape built directly in HBM, for benchmarks and tests
 * (no counterpart in the reference, which only loads converted checkpoints; its
 * converter quantizes through the gguf package, tools/convert_shieldstral_to_gguf.py).
 * Every matrix and token_embd is N(0, 0.02) and every norm gain N(1, 0.1), drawn from
 * a counter-based generator keyed by (seed, tensor, element) and quantized on the
 * device with the ggml block rules into weight_type / embd_type. */
shs_status shs_open_synthetic(const shs_config* cfg, int32_t weight_type, int32_t embd_type, uint64_t seed,
                              int32_t device, int32_t initial_capacity, shs_model** out);

/* Copies a model tensor back to the host: matrices in native GGUF block layout
 * (rows × row_bytes), norm gains as fp32. bytes must equal the tensor's size. */
shs_status shs_tensor_download(shs_model* model, const char* name, void* dst, size_t bytes);

void       shs_close(shs_model* model);
shs_status shs_get_config(const shs_model* model, shs_config* out);

/* KvCache (KvCache.cs:43-136) and MinistralModel.ResetKvCache (MinistralModel.cs:486). */
shs_status shs_kv_reset(shs_model* model);
shs_status shs_kv_length(const shs_model* model, int32_t* length);
shs_status shs_kv_capacity(const shs_model* model, int32_t* capacity);
/* KvCache.Snapshot (KvCache.cs:94-112): keys for every layer and head, then values,
 * each [layer][head][pos][dim]; n_floats must be 2·L·KVH·len·HD. */
shs_status shs_kv_snapshot(shs_model* model, int32_t length, float* dst, size_t n_floats);
/* KvCache.Restore (KvCache.cs:115-136): leaves the cache holding exactly that prefix. */
shs_status shs_kv_restore(shs_model* model, const float* src, size_t n_floats, int32_t length);

/* MinistralModel.ForwardAsync / ForwardSelectedAsync / PrefillAsync
 * (MinistralModel.cs:139-271). Appends tokens at the current KV length.
 *   head_mode 0 (PrefillAsync):        no head, logits_out unused
 *   head_mode 1 (ForwardSelectedAsync): logits_out[i] = logit of vocab_ids[i]
 *   head_mode 2 (ForwardAsync):         logits_out[0..vocab) for the last position
 * cancel_flag (may be NULL) is polled between layer launches; a cancelled pass
 * returns SHS_E_CANCELLED and leaves the KV length unchanged (MinistralModel.cs:240). */
shs_status shs_forward(shs_model* model, const int32_t* tokens, int32_t n_tokens, int32_t head_mode,
                       const int32_t* vocab_ids, int32_t n_ids, float* logits_out,
                       const volatile int32_t* cancel_flag);

/* Packed ragged prefill of independent prompts (no counterpart in the reference, which
 * runs them one ModerateAsync call at a time): sequence s is tokens[cu[s]..cu[s+1]),
 * positions restart at 0, attention is causal within the sequence, and
 * logits_out[s·n_ids + i] is sequence s's last-position logit of vocab_ids[i].
 * The model's KV cache is left untouched. */
shs_status shs_forward_batch(shs_model* model, const int32_t* tokens, const int32_t* cu_seqlens,
                             int32_t n_seq, const int32_t* vocab_ids, int32_t n_ids, float* logits_out);

/* IActivationSink (MinistralModel.cs:494-501): when set, every forward reports
 * embeddings, blk.{l}.{attn_norm,q_rope,k_rope,v,attn_weighted,attn_out,post_attn,
 * ffn_norm,ffn_out,output}, final_norm and (full head) logits as host fp32 rows×cols.
 * Capture serialises the pass; pass fn = NULL to turn it off. */
typedef void (*shs_capture_fn)(const char* name, const float* data, int32_t rows, int32_t cols, void* user);
shs_status shs_set_capture(shs_model* model, shs_capture_fn fn, void* user);

/* One decoder layer on a caller-supplied hidden state at positions 0..n-1 of an empty
 * cache (the body of the layer loop, MinistralModel.cs:214-238). x and y are host
 * [n × hidden] fp32; the KV cache is reset afterwards. No counterpart in the reference
 * API: the parity harness for a single layer. */
shs_status shs_layer_forward(shs_model* model, int32_t layer, const float* x, int32_t n_tokens, float* y);

/* ------------------------------------------------------ quantized matmul */

/* WeightMatrix.From + the integer GEMM of QuantMatMul (QuantMatMul.cs:292-410,
 * IntegerGemm.cs): a rows × cols weight in native block layout, uploaded once. */
shs_status shs_matrix_create(int32_t type, int32_t rows, int32_t cols, const void* data, int32_t device,
                             shs_matrix** out);
void       shs_matrix_free(shs_matrix* m);

/* QuantMatMul.ForwardAsync (QuantMatMul.cs:71-85): y[t][r] = x[t]·W[r] with x quantized
 * per 32-block to int8 (IntegerGemm.QuantizeActivations) and the per-block epilogue.
 * semantics 0 = IntegerGemm (fp32 scale, ties to even), 1 = IntegerDot's activation
 * quantization (fp16-rounded scale, half away from zero, IntegerDot.cs:60-98).
 * Host pointers: x [tokens × cols], y [tokens × rows]. */
shs_status shs_matmul(shs_matrix* m, const float* x, int32_t tokens, float* y, int32_t semantics);

/* QuantMatMul.ForwardRowsAsync (QuantMatMul.cs:98-110): only rows row_ids, bit-identical
 * to the same entries of shs_matmul. y [tokens × n_ids]. */
shs_status shs_matmul_rows(shs_matrix* m, const int32_t* row_ids, int32_t n_ids, const float* x,
                           int32_t tokens, float* y);

/* The exact int32 block sums I[t][r][b] = Σ_k (u−z)·q (IntegerGemm.cs:384-397) for
 * parity checks. out is host [tokens × rows × cols/32]. */
shs_status shs_matmul_block_sums(shs_matrix* m, const float* x, int32_t tokens, int32_t* out);

/* Device-pointer variant of shs_matmul for callers whose activations are already in
 * HBM (x_dev [tokens × cols] fp32, y_dev [tokens × rows] fp32). Runs on the matrix's
 * stream and returns when the result is written. */
shs_status shs_matmul_device(shs_matrix* m, const float* x_dev, int32_t tokens, float* y_dev);

/* No counterpart in the reference: shs_matmul_device for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments and bit-identical results; the activation codes go to a fixed
 * 16 MiB scratch array per GPU that the library holds until the process ends, so no
 * hipMalloc, hipFree or allocating call runs. tokens·(cols + cols/2) bytes, rounded up,
 * must fit in it (SHS_E_OUT_OF_RANGE otherwise: about 3600 tokens at 3072 columns).
 * Every call on a GPU shares that GPU's scratch: calls that overlap on one GPU (from
 * several threads or matrices) race and must be serialised by the caller. */
shs_status shs_matmul_device_noalloc(shs_matrix* m, const float* x_dev, int32_t tokens, float* y_dev);

/* e^x as the attention softmax and SwiGLU's sigmoid evaluate it on the device, for
 * x[0..n) → y (host buffers). Parity instrumentation: the CPU restatement performs the
 * same sequence of IEEE operations, and this entry lets a test compare them directly. */
shs_status shs_debug_expf(const float* x, int32_t n, float* y, int32_t device);

/* Blocks until every operation queued on the model's stream has completed. */
shs_status shs_synchronize(shs_model* model);

/* --------------------------------------------------------------- timing */

/* Per-kernel-class timing with HIP events recorded on the launching stream around
 * every launch of that class while enabled (no counterpart in the reference, whose
 * bench times whole calls, Benchmark.cs:537-611). Classes by step: gemm_qkv, gemm_o,
 * gemm_gate_up, gemm_down, gemm_head, gemv, attention, rmsnorm_quant, swiglu_quant,
 * quant_act, rope_store, embed; and by kernel, under the names rocprofv3 reports:
 * "k_gemm<type,TT,mode,BPS>" (each GEMM launch is in both), k_attn_scores, k_attn_softmax,
 * k_attn_pv, k_attn_fused. kernel_class "prefix*" sums the classes with that prefix.
 * total_ops is the algorithmic operation count (2·tokens·rows·cols for a GEMM), for
 * rmsnorm_quant the algorithmic HBM bytes (the rows read, their int8 codes and per-block
 * d, d·Σq and conversion column written), 0 where not counted. */
shs_status shs_profile_enable(shs_model* model, int32_t enable);
shs_status shs_profile_read(shs_model* model, const char* kernel_class, int64_t* launches,
                            double* total_ms, double* total_ops);
shs_status shs_profile_reset(shs_model* model);

#ifdef __cplusplus
}
#endif
#endif
