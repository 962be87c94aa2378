/*
 * oracle.h -- TEST INFRASTRUCTURE, NOT PRODUCT.
 *
 * A CPU restatement of the arithmetic tgo's batched forward pass performs,
 * written from the reference's Go sources (cited per function in oracle.c).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only as the checker or the timed CPU baseline. The product
 * (libtgohip.so) never links or calls it.
 *
 * Two layers:
 *   orc_*_f64   float64 restatements of tgo/internal/oracle (the reference
 *               every device result is judged against in tgo itself);
 *   orc_cpu_*   the f32 CPU path (tgo's CPU backend semantics: f32
 *               activations, weights dequantized to f32 on the fly, f32
 *               accumulate, f16 KV pool), OpenMP-parallel. This is what
 *               bench.py times as cpu_baseline ("port").
 *
 * Parity status of each function is stated in oracle.c's header.
 */
#ifndef TGO_ORACLE_H
#define TGO_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- seeded generators (shared definition with the product's synth) ---- */
uint64_t orc_splitmix64(uint64_t x);
uint64_t orc_hash3(uint64_t seed, uint64_t stream, uint64_t idx);
double   orc_normal(uint64_t seed, uint64_t stream, uint64_t idx);
void     orc_synth_normal_f32(uint64_t seed, uint64_t stream, size_t n, double sigma, float* out);
void     orc_synth_normal_f16(uint64_t seed, uint64_t stream, size_t n, double sigma, uint16_t* out);

/* ---- f16 conversion (weights/convert.go) ---- */
uint16_t orc_f32_to_f16_bits(float x, int* saturated);
float    orc_f16_to_f32(uint16_t h);
size_t   orc_to_f16(const float* src, uint16_t* dst, size_t n);
/* IEEE binary16 round-to-nearest-even with overflow to infinity and gradual
 * underflow: the device Cast (accel.ToFloat16) that narrows K/V rows. */
uint16_t orc_f32_to_f16_ieee(float x);
void     orc_f16_ieee_bits_array(const uint32_t* bits, uint16_t* out, size_t n);
void     orc_f16_loader_bits_array(const uint32_t* bits, uint16_t* out, size_t n);
void     orc_transpose(const float* src, float* dst, int rows, int cols);
int      orc_permute_heads(float* x, size_t n, int last_axis, int head_dim);

/* ---- quantized forms ---- */
void orc_quantize_int8(const float* w, size_t n, int8_t* q, uint16_t* scales);
void orc_dequant_int8(const int8_t* q, const uint16_t* scales, size_t n, float* out);
void orc_quantize_int4_tgo(const float* w, size_t n, uint32_t* codes, uint16_t* scales,
                           uint16_t* zeros);
void orc_dequant_int4_tgo(const uint32_t* codes, const uint16_t* scales, const uint16_t* zeros,
                          size_t n, float* out);
void orc_dequant_int4_sym(const uint32_t* qweight, const uint16_t* scales, int K, int N,
                          float* out);
void orc_synth_int4_sym(uint64_t seed, uint64_t stream, int K, int N, double sigma,
                        uint32_t* qweight, uint16_t* scales);
double orc_int4_tgo_bound(const float* x, const uint16_t* scales, const uint16_t* zeros,
                          int k, int n, int col);

/* ---- float64 oracle (internal/oracle) ---- */
void orc_rmsnorm_f64(const double* x, const double* gain, int rows, int width, double eps,
                     double* out);
void orc_matmul_f64(const double* x, const double* w, int m, int k, int n, double* out);
void orc_silu_f64(const double* x, int n, double* out);
void orc_swiglu_f64(const double* gate, const double* up, int n, double* out);
void orc_softmax_f64(const double* x, int n, double* out);
void orc_gather_rows_f64(const double* table, int vocab, int width, const int* ids, int n,
                         double* out);
void orc_rope_f64(const double* x, int rows, int width, int rotary, double base,
                  const int* pos, int style, double* out);
void orc_attention_f64(const double* q, const double* k, const double* v, int qseq, int qheads,
                       int kvheads, int headdim, int kvlen, double scale, int causal_base,
                       double* out);
/* Ragged paged attention over a paged cache: internal/conformance/ragged_test.go:151-208. */
void orc_ragged_attention_f64(const float* q, int T, int H, int Hkv, int dh,
                              const uint16_t* k_f16, const uint16_t* v_f16,
                              const float* k_f32, const float* v_f32,
                              int B, const uint32_t* lengths, const uint32_t* extents,
                              const uint32_t* pages, int max_pages, int block, double scale,
                              double* out, double* budget3);

/* ---- f32 CPU path (tgo's CPU backend semantics) ---- */
typedef struct orc_model orc_model;
enum { ORC_FORM_F16 = 0, ORC_FORM_I8 = 1, ORC_FORM_I4_TGO = 2, ORC_FORM_I4_SYM = 3 };
orc_model* orc_model_new(int layers, int hidden, int heads, int kv_heads, int head_dim,
                         int ffn, int vocab, float eps, float theta, int block, int capacity);
void orc_model_free(orc_model*);
int  orc_model_weight(orc_model*, const char* port, int form, int K, int N, const void* plane,
                      const void* scales, const void* zeros);
int  orc_model_gain(orc_model*, const char* port, const float* g, int width);
/* Synthesize every weight of the model from (seed, form) exactly as the
 * product's synthesizer does; layers_limit < 0 means all layers. */
int  orc_model_synth(orc_model*, uint64_t seed, int form, double sigma, int layers_limit);
void orc_model_kv(orc_model*, uint16_t** k, uint16_t** v);
/* The synthesizer's gains: multiples of 1/8 in [-2, 2) from (seed, stream). */
void orc_synth_gain(uint64_t seed, uint64_t stream, size_t n, float* out);
/* Planted mistakes for the sensitivity tests (0 = none). */
enum {
  ORC_FAULT_NONE = 0,
  ORC_FAULT_QKNORM_AFTER_ROPE = 1, /* q/k RMSNorm applied after RoPE */
  ORC_FAULT_QK_UNIT_GAIN = 2,      /* q/k-norm gain dropped */
  ORC_FAULT_K_TAKES_Q_GAIN = 3,    /* k rows normalized with the q gain */
  ORC_FAULT_QK_GAIN_AFTER_ROPE = 4,/* normalized, rotated, then scaled by the gain */
  ORC_FAULT_NORM_UNIT_GAIN = 5,    /* attn_norm / ffn_norm gains dropped */
  ORC_FAULT_FINAL_UNIT_GAIN = 6    /* final_norm gain dropped */
};
int  orc_model_set_fault(orc_model*, int fault);
/* One batched step: ports as model.NewBatchStep packs them (model/batch.go). Writes
 * logits [B,V] (rows of members with extent 0 are written as zeros). layers < 0: all. */
int  orc_model_step(orc_model*, int rows, int B, const uint32_t* ids, const uint32_t* posq,
                    const uint32_t* posk, const uint32_t* slots, const uint32_t* lengths,
                    const uint32_t* extents, const uint32_t* last, const uint32_t* pages,
                    int max_pages, float* logits, int layers);
/* The f32 CPU path's attention alone (f16 cache, f32 accumulate). */
void orc_cpu_ragged_attention(const float* q, int T, int H, int Hkv, int dh,
                              const uint16_t* kc, const uint16_t* vc, int B,
                              const uint32_t* lengths, const uint32_t* extents,
                              const uint32_t* pages, int max_pages, int block, float scale,
                              float* out);
/* The f32 CPU path's projection alone: y[M,N] = x[M,K] deq(W). */
int  orc_cpu_linear(const float* x, int M, int K, int N, int form, const void* plane,
                    const void* scales, const void* zeros, float* y);
int  orc_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
