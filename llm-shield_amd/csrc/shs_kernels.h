// Internal interface between the host runtime (shs_api.cpp) and the gfx950 kernels
// (shs_kernels.hip). Device layouts are described once here.
//
// Repacked weight matrix (rows padded to a multiple of 32, B = cols/32 blocks):
//   record (tile, b) for 32 consecutive rows × one 32-wide block:
//     qs  [tiles][B][32 rows][QSB]  QSB = 16 (4/5-bit types; GGUF nibble order kept)
//                                   QSB = 32 (Q8_0; bytes permuted like activations)
//     qh  [tiles][B][32 rows] u32   fifth bits (Q5_0/Q5_1), GGUF bit order kept
//     d   [tiles][B][32 rows] f32   block scale, fp16 widened exactly
//     m   [tiles][B][32 rows] f32   block min (Q4_1/Q5_1)
// Quantized activations (T padded to Tpad, a multiple of 32):
//     q   [Tpad/32][B][2 halves][32 tokens][16 int8]  half h of a token's block holds the
//                                          elements [8h..8h+7, 16+8h..16+8h+7] — the 16 bytes
//                                          lane half h of the int8 MFMA multiplies, in the order
//                                          the weight nibbles unpack to
//     d   [B][Tpad] f32   scale max|x|/127
//     cv  [B][Tpad] 8 B   the block's conversion operand: fp16 (−6144, −⌊Σq/64⌋, −(Σq mod 64), 0)
//                         — the B column of the fp16 MFMA that turns the integer MFMA's offset
//                         sums into exact fp32 block sums (see k_gemm)
//     ds  [B][Tpad] f32   RN(d·float(Σq)) — the offset types' second factor
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace shs {

enum { SHS_TYPE_F32 = 0, SHS_TYPE_F16 = 1, SHS_TYPE_Q4_0 = 2, SHS_TYPE_Q4_1 = 3,
       SHS_TYPE_Q5_0 = 6, SHS_TYPE_Q5_1 = 7, SHS_TYPE_Q8_0 = 8 };

struct DevMatrix {
    int type = -1, rows = 0, cols = 0, blocks = 0, tiles = 0;
    uint8_t* qs = nullptr;
    uint32_t* qh = nullptr;
    float* d = nullptr;
    float* m = nullptr;
};

struct ActQ8 {
    int T = 0, Tpad = 0, K = 0, B = 0;
    int8_t* q = nullptr;
    float* d = nullptr;
    uint2* cv = nullptr;
    float* ds = nullptr;
};

// The four arrays of an ActQ8 live in one allocation, in this order, each 256-byte
// aligned: codes [Tpad·K], d_a and d_a·Σq [Tpad·B] fp32, conversion columns [Tpad·B]. The
// GEMM addresses all of them from the codes' base with 32-bit offsets.
inline size_t act_q8_round(size_t v) { return (v + 255) & ~(size_t)255; }
inline size_t act_q8_bytes(int T, int K)
{
    const size_t Tpad = ((size_t)T + 31) / 32 * 32, B = (size_t)K / 32;
    return act_q8_round(Tpad * K) + 2 * act_q8_round(4 * Tpad * B) + act_q8_round(8 * Tpad * B);
}
inline ActQ8 act_q8_view(void* base, int T, int K)
{
    ActQ8 a;
    a.T = T;
    a.Tpad = (T + 31) / 32 * 32;
    a.K = K;
    a.B = K / 32;
    const size_t qb = act_q8_round((size_t)a.Tpad * K), fb = act_q8_round(4 * (size_t)a.Tpad * a.B);
    uint8_t* p = static_cast<uint8_t*>(base);
    a.q = reinterpret_cast<int8_t*>(p);
    a.d = reinterpret_cast<float*>(p + qb);
    a.ds = reinterpret_cast<float*>(p + qb + fb);
    a.cv = reinterpret_cast<uint2*>(p + qb + 2 * fb);
    return a;
}

// One attention work item: q_count ≤ 32 queries of one sequence at rows q_start.. of q/ctx,
// the first at position pos0, attending to cache indices key_start .. key_start + pos0 +
// q_count − 1 (query i sees pos0 + i + 1 keys). Scores of the item's heads go to scratch + s_off.
struct AttnItem {
    int q_start, q_count, key_start, pos0;
    int64_t s_off;  // float offset of the item's score tiles: n_kv · 4 · n_tiles tiles of 1024 floats
};

// A run of ≤ 4 key tiles of one item, the unit of the score kernel.
struct AttnChunk {
    int item, kt0, nkt, pad;
};

// GEMM_SWIGLU: the fused gate|up matrix (n_ft feature tiles of gate rows, then the same of
// up rows) with Kernels.SwiGlu and the down projection's 32-block quantization applied in
// the epilogue; the output is the down projection's activation codes.
// GEMM_QKV: the fused q|k|v matrix with RoPE (and the query position scale) applied in the
// epilogue; q goes to the output, k and v to the KV cache (RopeArgs).
enum GemmMode { GEMM_STORE = 0, GEMM_ADD = 1, GEMM_SWIGLU = 2, GEMM_QKV = 3 };

// RoPE and KV-cache placement for the GEMM_QKV epilogue and k_rope_store: token t sits at
// position pos[t] and cache slot slot0 + t; tables are [position][half] (cos, sin) and
// [position] (query scale).
struct RopeArgs {
    const int32_t* pos = nullptr;
    const float* ct = nullptr;
    const float* st = nullptr;
    const float* qscale = nullptr;
    int half = 0, n_head = 0, n_kv = 0, hd = 0;
    float* kc = nullptr;
    float* vc = nullptr;
    int cap = 0, slot0 = 0;
};

// The input of a narrow q|k|v or gate|up GEMM given as the hidden rows instead of codes:
// every work-group applies Kernels.RmsNorm with gain w to rows x (T of them, stride ldx)
// and quantizes the result itself, while its weight loads are in flight — the same
// arithmetic as k_rmsnorm_quant, so the codes are the same bits.
struct NormIn {
    const float* x = nullptr;
    int ldx = 0;
    const float* w = nullptr;
    float eps = 0.0f;
};

int qs_bytes(int type);
bool type_supported(int type);
bool type_has_offset(int type);
bool type_has_qh(int type);

// All launchers return hipError_t of the launch.
hipError_t launch_repack(const DevMatrix& m, const uint8_t* native, int row0, int nrows, hipStream_t s);
hipError_t launch_quant_act(const float* x, int ldx, const ActQ8& a, int semantics, hipStream_t s);
hipError_t launch_rmsnorm_quant(const float* x, int ldx, const float* w, float eps, int n, const ActQ8& a,
                                float* y_opt, hipStream_t s);
hipError_t launch_swiglu_quant(const float* gu, int ldgu, int ffn, const ActQ8& a, float* y_opt, hipStream_t s);
hipError_t launch_gemm(const DevMatrix& w, const ActQ8& a, float* y, int ldy, int mode, hipStream_t s);
// y = SwiGLU(x·[gate|up]ᵀ) quantized into `out` (K = 32·n_ft); w holds 2·n_ft row tiles.
hipError_t launch_gemm_swiglu(const DevMatrix& w, const ActQ8& a, int n_ft, const ActQ8& out, hipStream_t s,
                              const NormIn* norm = nullptr);
// q|k|v = x·Wᵀ with RoPE: rotated (and scaled) q into y, rotated k and v into the cache.
hipError_t launch_gemm_qkv(const DevMatrix& w, const ActQ8& a, float* y, int ldy, const RopeArgs& ra, hipStream_t s,
                           const NormIn* norm = nullptr);
// The token tiles per block launch_gemm picks for this shape (the k_gemm instantiation's TT).
int gemm_token_tiles(const DevMatrix& w, const ActQ8& a, int mode);
// Blocks per K-loop stage of that instantiation (its BPS): single-tile Q4_0 work-groups take
// 4 when the block count is a multiple of 4 (three 16 KB slots, so three work-groups still
// share a CU; the other types' larger slots would leave room for two), everything else 2.
inline int gemm_stage_blocks(const DevMatrix& w, int token_tiles)
{
    return token_tiles == 1 && w.type == SHS_TYPE_Q4_0 && w.blocks % 4 == 0 ? 4 : 2;
}
// Up to NARROW_MAX_T tokens, launch_gemm, launch_gemm_qkv and launch_gemm_swiglu stream the
// weights through k_gemm_narrow instead (same epilogues); returns the token count when they
// do for this mode, else 0. With `with_norm`, whether the kernel can also form its input
// itself (NormIn).
enum { NARROW_MAX_T = 4 };
int gemm_narrow_tokens(const DevMatrix& w, const ActQ8& a, int mode, bool with_norm = false);

hipError_t launch_gemm_block_sums(const DevMatrix& w, const ActQ8& a, int32_t* out, hipStream_t s);
hipError_t launch_gemv_rows(const DevMatrix& w, const ActQ8& a, const int32_t* row_ids, int n_ids, float* y,
                            hipStream_t s);
hipError_t launch_embed(const DevMatrix& table, const int32_t* ids, int n, float* h, int ldh, hipStream_t s);
hipError_t launch_rope_store(float* qkv, int ldqkv, int T, int n_head, int n_kv_head, int head_dim,
                             const int32_t* pos, const float* cos_tab, const float* sin_tab,
                             const float* qscale_tab, int half, float* kc, float* vc, int cap,
                             int kv_slot0, hipStream_t s);
// Causal GQA attention: the scores, then either the fused softmax + values kernel or the
// softmax and values launches; the softmax launch clears the two work counters
// (counters[0..1]) it and the values launch share.
hipError_t launch_attn_scores(const float* q, int ldq, const float* kc, int cap, const AttnItem* items,
                              const AttnChunk* chunks, int n_chunks, int n_head, int n_kv, int head_dim, float scale,
                              float* scratch, float* pm, hipStream_t s);
// Blocks of the score kernel resident on the whole device (per CU × n_cu).
int attn_score_slots(int n_cu);
hipError_t launch_attn_softmax(const AttnItem* items, int n_items, int n_head, int n_kv, float* scratch, const float* pm,
                               int* counters, int n_cu, hipStream_t s);
// ctx, or with `codes` set, ctx quantized per 32-dimension block straight into the o
// projection's activation codes (rows of items only; ctx is then not written).
hipError_t launch_attn_pv(const float* vc, int cap, const AttnItem* items, int n_items, int n_head, int n_kv,
                          const float* scratch, float* ctx, int ldc, const ActQ8* codes, int* counters, int n_cu,
                          hipStream_t s);
// Scores, softmax and values in one kernel (in place of the three above): one block per
// (item, query head) holds the item's first kt_cap score tiles in its LDS; kt_cap at most
// attn_fused_kt_limit(the device's LDS per block). When an item has more key tiles, `spill`
// (the scratch regions place_items lays out) holds its later tiles; with spill null every
// item must fit kt_cap tiles. Items of up to ATT_FUSED_MAX_KT key tiles take it; longer ones
// the three kernels above.
constexpr int ATT_FUSED_MAX_KT = 256;
hipError_t launch_attn_fused(const float* q, int ldq, const float* kc, const float* vc, int cap, const AttnItem* items,
                             int n_items, int n_head, int n_kv, int head_dim, float scale, float* ctx, int ldc,
                             const ActQ8* codes, int kt_cap, float* spill, hipStream_t s);
int attn_fused_kt_limit(int max_lds_bytes);
// Attention for items of at most ATT_DEC_MAX_Q queries (decode), at most 4 query heads per
// KV head: a score kernel over (item, KV head, 64-key chunk) writing the scores to the
// scratch (each item's region from place_items), then softmax + values over (item, query
// head, 32-dimension slice). Every item must have at most max_qc queries and max_keys keys,
// max_keys at most attn_decode_max_keys(max_qc, the device's LDS per block). ctx, or with
// `codes` set, the o projection's codes of the items' rows.
enum { ATT_DEC_MAX_Q = 4 };
int attn_decode_max_keys(int max_qc, int max_lds_bytes);
hipError_t launch_attn_decode(const float* q, int ldq, const float* kc, const float* vc, int cap, const AttnItem* items,
                              int n_items, int n_head, int n_kv, int head_dim, float scale, int max_qc, int max_keys,
                              float* scratch, float* ctx, int ldc, const ActQ8* codes, hipStream_t s);
hipError_t launch_expf(const float* x, int n, float* y, hipStream_t s);
hipError_t launch_copy_rows(const float* src, int lds, float* dst, int ldd, int rows, int cols, hipStream_t s);
hipError_t launch_fill_zero(float* p, size_t n, hipStream_t s);
hipError_t launch_add_inplace(float* a, const float* b, size_t n, hipStream_t s);
hipError_t launch_gather_rows(const float* src, int lds, const int32_t* rows, int n, int cols, float* dst, int ldd,
                              hipStream_t s);

// Synthetic random-init weights: N(mean, std) from a counter-based generator keyed by
// (seed, tensor id, element), quantized with the ggml block rules into native layout.
hipError_t launch_synth_native(int type, uint64_t seed, uint64_t tensor_id, int rows, int cols, float mean, float std,
                               uint8_t* native, hipStream_t s);
hipError_t launch_synth_f32(uint64_t seed, uint64_t tensor_id, int64_t n, float mean, float std, float* out,
                            hipStream_t s);
// Inverse of launch_repack: rows [0, rows) back to native GGUF blocks.
hipError_t launch_unpack_native(const DevMatrix& m, int row0, int nrows, uint8_t* native, hipStream_t s);

// Fixed device scratch for callers that cannot allocate: one array of this many bytes per
// GPU, in the code object, held until the process ends. noalloc_scratch() returns the
// array's device address on `device` (looked up once per device with that device made
// current, then cached); host code uses only that address, never the array's name.
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(16) << 20;
hipError_t noalloc_scratch(int device, uint8_t** out);

}  // namespace shs
