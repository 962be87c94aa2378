/*
 * tgohip.h -- C ABI of libtgohip.so, the MI355X (gfx950) implementation of
 * tgo's batched forward-pass hot path.
 *
 * tgo (github.com/latere-ai/tgo) records its forward pass as accel operators
 * and hands the graph to golang.design/x/accel. This library replaces that
 * boundary for the batched path: the ops of one continuous-batching step
 * (model/qwen3_graph.go:32-128) run as hand-written HIP kernels behind the
 * entry points below. Each entry point names the reference interface it
 * replaces (file:line in the reference tree).
 *
 * Conventions (inherited from the reference):
 *   - Every call returns 0 on success or a negative TGOHIP_E* code; the
 *     message naming the offending field is tgohip_last_error() (thread
 *     local). Refusals are loud, never clamps (model/batch.go:67-125).
 *   - Out-of-range data that the reference defines is not an error: a slot
 *     at or past the pool capacity is a dropped write (plan.go:182-192), and
 *     a query row past the sum of the extents is inert (its output is zero).
 *   - Pointers documented "host" are host memory; "device" pointers are HIP
 *     device memory on the context's device. Sizes are elements unless named
 *     *_bytes.
 *   - One context is one device and one stream; calls on a context are
 *     serialised by the caller (tgo serialises under Model.mu,
 *     model.go:114-127).
 */
#ifndef TGOHIP_H
#define TGOHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define TGOHIP_OK 0
#define TGOHIP_EINVAL (-1)   /* an argument is refused; the message names it */
#define TGOHIP_ENOMEM (-2)   /* a device allocation failed */
#define TGOHIP_EDEVICE (-3)  /* a HIP call failed */
#define TGOHIP_ESTATE (-4)   /* the context is not configured for this call */
#define TGOHIP_EEXHAUSTED (-5) /* prefix.ErrExhausted (internal/prefix/prefix.go:54) */
#define TGOHIP_ENOSLOT (-6)  /* tgo.ErrNoSlot (scheduler.go:175) */

/* Weight forms: nn.Form (nn/nn.go:118-136), plus the BASELINE int4 pack. */
#define TGOHIP_FORM_F16 0     /* [K,N] f16 row-major */
#define TGOHIP_FORM_I8 1      /* i8 [K,N] + f16 scale per 32 flattened elements */
#define TGOHIP_FORM_I4_TGO 2  /* u32 codes [ceil(KN/8)], element i of a word in bits
                                 4i..4i+3; f16 scale and f16 zero per 128 flattened
                                 elements; w = (q - z) * s */
#define TGOHIP_FORM_I4_SYM 3  /* symmetric int4, group 32 along K: u32 [K/8][N], word
                                 (r,n) holds k=8r+i in bits 4i..4i+3 as q+8; f16
                                 scales [K/32][N]; w = q * s */

/* Activation / output dtypes */
#define TGOHIP_F32 0
#define TGOHIP_F16 1
/* An f32 activation [M,K] already split for tgo's arithmetic (precision mode 1):
 * the f16 plane hi = f16(x) [M,K] followed by the f16 plane lo = f16(x - hi)
 * [M,K]; the same bytes as f32. tgohip_linear's x_dtype only. */
#define TGOHIP_F16X2 2

const char* tgohip_last_error(void);
const char* tgohip_version(void);

/* ---- context: replaces accel.OpenBest/Device/Queue (model.go:368-387) --- */
typedef struct tgohip_ctx tgohip_ctx;

/* Opens device `device` and creates the context's stream. NULL on failure. */
tgohip_ctx* tgohip_open(int device);
/* Synchronises, frees every device allocation the context owns, and closes it
 * (close order of weights/weights.go:349-371, model.go:338-365). */
void tgohip_close(tgohip_ctx* ctx);
/* The stream the context launches on (a hipStream_t), for callers that time
 * kernels with events on that stream. */
void* tgohip_stream(tgohip_ctx* ctx);
int tgohip_sync(tgohip_ctx* ctx);
/* Launch on a caller's stream (a hipStream_t, e.g. torch's current stream)
 * instead of the context's own. NULL is the device's default stream. The
 * context's own stream is a blocking stream (ordered against the default
 * stream); tgohip_use_own_stream returns to it. */
int tgohip_set_stream(tgohip_ctx* ctx, void* stream);
int tgohip_use_own_stream(tgohip_ctx* ctx);
/* Arithmetic of the step. 1 (the default) is tgo's CPU path (nn/blocks.go:13-21): every
 * projection multiplies the f32 activation (carried as an f16 high + low pair,
 * ~22 bits) by the unrounded dequantized weight, f32 accumulate: symmetric
 * int4 as the exact codes with each 32-k group's scale applied in f32 (two
 * f16 MFMAs per product), the other forms as an exact f16 high + low weight
 * pair (three) -- and attention weights V by the f32 softmax probabilities
 * (hi + lo); logits stay within 2e-3 of tgo's CPU path through every layer of
 * the 8B and 32B shapes. 0 rounds activations, weights and probabilities to
 * f16 for one MFMA each: 1.6-2.2x faster, with an f16 storage error per
 * operand that grows with depth (about 5e-3 of the row's largest logit after
 * 36 layers). */
int tgohip_set_precision(tgohip_ctx* ctx, int mode);
/* Prefix-shared (cascade) attention, the "read a shared page once" design of
 * tgo's prefix cache (internal/prefix block sharing; specs/016-prefix-cache.md).
 * No counterpart in the reference's kernels: tgo reads a shared page once per
 * sequence. With min_sharers >= 2, decode rows of sequences whose page tables
 * begin with the same pages (at least 64 positions, whole 64-position tiles
 * visible to every row) attend to that shared prefix in one pass per group of
 * up to 128/G sequences, and their own suffixes separately; the parts merge
 * in a fixed order. 0 (the default) turns it off: every sequence is then
 * decomposed as it would be alone, bit-for-bit (ragged_test.go:295), which a
 * grouped prefix cannot promise (its results differ from the ungrouped ones
 * within f32 rounding). */
int tgohip_set_cascade(tgohip_ctx* ctx, int min_sharers);

/* ---- model configuration: replaces model.Config (model/config.go) -------- */
typedef struct {
  int32_t layers, hidden, heads, kv_heads, head_dim, ffn, vocab;
  float rms_eps;    /* rms_norm_eps (fixture_test.go:95) */
  float rope_theta; /* rope_theta, bound as the f32 scalar rope_base (batch.go:507-510) */
  int32_t block;    /* positions per KV page (blocks.go:28 CacheBlock; a parameter here) */
} tgohip_model_cfg;

int tgohip_config(tgohip_ctx* ctx, const tgohip_model_cfg* cfg);
/* The configuration a context was given (for a loader that walks its ports). */
int tgohip_get_config(tgohip_ctx* ctx, tgohip_model_cfg* cfg);

/* Uploads one weight port, as nn.Graph.Weight declares it (nn/nn.go:209-259)
 * and weights.Load binds it (weights/weights.go:629-743, model.go:489-543).
 * port: "embed" [V,d], "lm_head" [d,V], "<l>.wq|wk|wv|wo|wgate|wup|wdown"
 * [K,N] already transposed and q/k-permuted. plane/scales/zeros are host
 * memory in the form's layout (scales NULL for F16, zeros NULL unless
 * I4_TGO). The library repacks into its device layout. The embedding may be
 * F16 or I8 (QuantGatherRows, model/qwen3_graph.go:57-61). */
int tgohip_weight(tgohip_ctx* ctx, const char* port, int form, int K, int N,
                  const void* plane, const void* scales, const void* zeros);
/* tgohip_weight from an f32 plane, quantized on the device: weights.Load's
 * quantize-then-upload of a projection or of the int8-capped embedding
 * (weights/weights.go:694-743; quantizeInto, weights/convert.go:206-217).
 * w: host [K,N] f32 (already transposed and q/k-permuted); form I8 or I4_TGO.
 * The device codes, scales and zeros equal tgohip_quantize_int8 /
 * tgohip_quantize_int4's on the same plane, bit for bit (NaN, infinities and
 * values past f16's range included), so the result is that of those calls
 * followed by tgohip_weight; the quantization runs at device speed instead of
 * one f64 division per element on the host. */
int tgohip_weight_f32(tgohip_ctx* ctx, const char* port, int form, int K, int N, const float* w);
/* Uploads an f32 norm gain (nn/nn.go:266-274, gains.go:40-69):
 * "<l>.attn_norm|ffn_norm" [d], "<l>.qnorm|knorm" [d_h], "final_norm" [d]. */
int tgohip_gain(tgohip_ctx* ctx, const char* port, const float* g, int width);
/* Synthesises every weight port on the device from a seed (random init for
 * benchmarks; bit-identical to the CPU restatement's synthesizer). form is the
 * projections' form; the embedding is F16 under F16 and I8 otherwise. */
int tgohip_synth_weights(tgohip_ctx* ctx, uint64_t seed, int form, double sigma);

/* Allocates the shared KV pool: K and V f16 [layers, positions, kv_heads,
 * head_dim], zeroed (blocks.go:74-139). positions is rounded down to whole
 * pages. Any earlier pool is released first; if the device refuses the new
 * one (TGOHIP_ENOMEM) the context holds no pool until a later call succeeds. */
int tgohip_kv_alloc(tgohip_ctx* ctx, int positions);
/* Device pointers of the K and V pools and their capacity in positions. */
int tgohip_kv_pointers(tgohip_ctx* ctx, void** k, void** v, int* positions);

/* ---- one batched step: replaces Batch.step's WriteBuffer x8 + Submit +
 *      Wait + ReadBuffer (batch.go:384-437) -------------------------------- */
typedef struct {
  int32_t rows;              /* plan rows T >= sum(extents) */
  int32_t batch;             /* B members */
  int32_t max_pages;         /* page-table width */
  const uint32_t* ids;       /* host [rows]        model.BatchStep.IDs */
  const uint32_t* posq;      /* host [rows*H]      .PosQ  (or NULL, see below) */
  const uint32_t* posk;      /* host [rows*H_kv]   .PosK  (or NULL) */
  const uint32_t* slots;     /* host [rows]        .Slots (or NULL) */
  const uint32_t* lengths;   /* host [B]           .Lengths */
  const uint32_t* extents;   /* host [B]           .Extents */
  const uint32_t* last;      /* host [B]           .Last */
  const uint32_t* pages;     /* host [B*max_pages] page table (batch.go:397-402) */
} tgohip_batch_step;

typedef struct {
  double submit_ms;   /* pack + upload + enqueue (bench/bench.go:60-74 "submit") */
  double device_ms;   /* first kernel to last kernel, HIP events ("device") */
  double readback_ms; /* logits / token ids back to the host ("readback") */
} tgohip_timings;

/* Runs the whole forward pass for one step. logits_out: host [B,V] f32 or
 * NULL; rows of members with extent 0 are zero. argmax_out: host [B] int32 or
 * NULL: the greedy token per member (sample/stages.go:196-206, first strict
 * maximum; -1 for extent 0). timings may be NULL.
 * posq, posk and slots may all be NULL (no counterpart in tgo, whose
 * NewBatchStep packs them, batch.go:310-340): the device derives them from the
 * members, the values NewBatchStep would pack. Row t belongs to the last member
 * b with cu_b <= t (cu: prefix sums of extents) and sits at position
 * p = lengths[b] - extents[b] + (t - cu_b), slot pages[b][p / block] * block +
 * p % block; rows past sum(extents) repeat the last member's last position
 * with slot = capacity. Only ids and the per-member ports then cross PCIe.
 * Padding rows (t >= sum(extents), a bucket's rows: batch.go:362-366) are not
 * computed when they cannot change anything: every padding row's slot is at
 * or past capacity (its K/V write is dropped, plan.go:180-192) and no member
 * with a nonzero extent reads its logits from one. A step bucketed from 1152
 * to 2048 rows then costs the 1152 rows. Otherwise every row runs. */
int tgohip_step(tgohip_ctx* ctx, const tgohip_batch_step* step, float* logits_out,
                int32_t* argmax_out, tgohip_timings* timings);

/* The top-two margin of each of the last step's B members, computed on the
 * device in the argmax pass: TopTwoMargin (internal/conformance/measure.go:91),
 * the largest logit minus the second largest in float64, 0 for a repeated
 * maximum. out: host [B] double. Waits for the step. */
int tgohip_step_margins(tgohip_ctx* ctx, double* out, int B);

/* ---- op-level entry points (isolated configs and unit parity) ----------- */

/* tensor.Attention, ragged + paged + f16 cache (nn/attention.go:234-253;
 * internal/conformance/ragged_test.go:251-257). Device pointers: q [T,H,d_h]
 * (q_dtype), k/v [C, H_kv, d_h] f16 (one layer's pool view), out [T,H,d_h]
 * (out_dtype). Host pointers: lengths/extents [B], pages [B*max_pages].
 * Token i of sequence s (flat row cu_s+i) sits at position L_s-n_s+i and
 * attends to positions 0..L_s-n_s+i; rows >= sum(extents) are written zero. */
int tgohip_paged_attention(tgohip_ctx* ctx, const void* q, int q_dtype, int T, int H,
                           int H_kv, int head_dim, const void* k, const void* v,
                           int capacity, int B, const uint32_t* lengths,
                           const uint32_t* extents, const uint32_t* pages, int max_pages,
                           int block, float scale, void* out, int out_dtype);

/* The same launch planned once and replayed `iters` times with the metadata
 * resident (timing helper; each replay is the kernels alone). */
int tgohip_paged_attention_replay(tgohip_ctx* ctx, const void* q, int q_dtype, int T, int H,
                                  int H_kv, const void* k, const void* v, int capacity, int B,
                                  const uint32_t* lengths, const uint32_t* extents,
                                  const uint32_t* pages, int max_pages, int block, float scale,
                                  void* out, int out_dtype, int iters);

/* Greedy selection over device logits [B,V] f32: ids[b] (device int32) is the
 * first index of the strict maximum of row b, the argmax of
 * sample/stages.go:196-206 (a NaN is never taken after index 0; NaN at index 0
 * gives 0). margins (device [B] double, or NULL): TopTwoMargin of each row
 * (internal/conformance/measure.go:91-110), which seeds with x[0], x[1] and
 * takes later values by strict comparison. V >= 2. */
int tgohip_greedy(tgohip_ctx* ctx, const float* logits, int B, int V, int32_t* ids,
                  double* margins);

/* Uploads a weight for tgohip_linear under a handle (any form above). */
int tgohip_weight_upload(tgohip_ctx* ctx, int form, int K, int N, const void* plane,
                         const void* scales, const void* zeros, int* handle);
/* tgohip_weight_upload from an f32 [K,N] host plane quantized on the device
 * (I8 or I4_TGO), as tgohip_weight_f32 does for a port. */
int tgohip_weight_upload_f32(tgohip_ctx* ctx, int form, int K, int N, const float* w, int* handle);
/* Synthesises a [K,N] weight of `form` on the device under a handle, from
 * (seed, stream) as tgohip_synth_weights does for a port. */
int tgohip_weight_synth(tgohip_ctx* ctx, int form, int K, int N, uint64_t seed, uint64_t stream,
                        double sigma, int* handle);
int tgohip_weight_free(tgohip_ctx* ctx, int handle);

/* nn.Linear (nn/blocks.go:22-46): y[M,N] = x[M,K] . deq(W)[K,N], f32
 * accumulate. x device [M,K] (x_dtype), y device [M,N] (y_dtype). With x_dtype
 * F32 or F16X2 the product is tgo's arithmetic (the f32 activation times the
 * unrounded dequantized weight); with F16, the f16 activation times the
 * dequantized weight rounded to f16. */
int tgohip_linear(tgohip_ctx* ctx, int handle, const void* x, int x_dtype, int M, void* y,
                  int y_dtype);

/* tgohip_linear without allocating device memory. No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The caller
 * passes x and y; the split-K partials go to a static 64 MiB device array (one
 * per GPU, held until the process ends) instead of the context's workspace.
 * Same kernels and splits as tgohip_linear, so the same result. A call whose
 * partials need more than 64 MiB is refused (TGOHIP_EINVAL). Every call on a
 * GPU shares that GPU's array: calls that overlap on one GPU (two streams or
 * two contexts at once) race; calls in stream order do not. */
int tgohip_linear_noalloc(tgohip_ctx* ctx, int handle, const void* x, int x_dtype, int M,
                          void* y, int y_dtype);
/* Bytes of split-K partials a linear call over M rows of a handle's weight
 * with activations of x_dtype (TGOHIP_F16, TGOHIP_F32 or TGOHIP_F16X2) needs:
 * 0 when it runs unsplit. tgohip_linear_noalloc refuses calls above 64 MiB. */
int tgohip_linear_workspace(tgohip_ctx* ctx, int handle, int x_dtype, int M, size_t* bytes);

/* Dequantizes a handle's weight to f32 [K,N] on the device exactly as the
 * host restatement does ((q - z) * s in f32). y: device [K,N] f32. */
int tgohip_dequant(tgohip_ctx* ctx, int handle, float* y);
/* The values the MFMA path multiplies: the dequantized weight rounded once
 * to f16 (round to nearest even). y: device [K,N] f16. */
int tgohip_dequant_f16(tgohip_ctx* ctx, int handle, uint16_t* y);

/* ---- host-side mirrors of the reference's batched path ------------------ */

/* model.NewBatchStep (model/batch.go:66-152). Members are given as
 * concatenated tokens with per-member counts, first positions and page rows
 * of width max_pages (pages_len[i] entries valid). Outputs are host arrays
 * sized rows, rows*H, rows*H_kv, rows, B, B, B. */
int tgohip_new_batch_step(int vocab, int heads, int kv_heads, int rows, int B,
                          const int32_t* tokens, const int32_t* counts, const int32_t* first,
                          const int32_t* pages, const int32_t* pages_len, int max_pages,
                          int block, int capacity, uint32_t* ids, uint32_t* posq,
                          uint32_t* posk, uint32_t* slots, uint32_t* lengths,
                          uint32_t* extents, uint32_t* last);

/* nextStep (schedule.go:80-118) over n slots described by arrays:
 * live[n], prompt_len[n], prefilled[n]. Outputs work_slot/work_start/
 * work_count (at most n entries; start is the prompt offset for a prefill
 * and -1 for a decode), the entry count, and the prefill/decode totals. */
int tgohip_next_step(int n, const int32_t* live, const int32_t* prompt_len,
                     const int32_t* prefilled, int chunk, int rows, int32_t* work_slot,
                     int32_t* work_start, int32_t* work_count, int32_t* n_work,
                     int32_t* prefill, int32_t* decode);
/* victim (schedule.go:132-150): -1 when nothing is live. */
int tgohip_victim(int n, const int32_t* live, const int32_t* prompt_len,
                  const int32_t* prefilled, const uint64_t* arrived);

/* SHA-256 (FIPS 180-4) of a byte string: the hash the prefix chain uses
 * (internal/prefix/hash.go:46-65). */
int tgohip_sha256(const void* data, size_t n, uint8_t* out32);

/* prefix.Pool / prefix.Lease (internal/prefix/prefix.go, lease.go). */
typedef struct tgohip_pool tgohip_pool;
typedef struct tgohip_lease tgohip_lease;
tgohip_pool* tgohip_pool_new(int block, int blocks, int scope);
void tgohip_pool_free(tgohip_pool* p);
/* stats: acquires, hits, reused, prompt, evictions, publishes, adoptions,
 * in_use, cached, free */
void tgohip_pool_stats(tgohip_pool* p, int64_t* stats10);
int tgohip_pool_acquire(tgohip_pool* p, const int32_t* ids, int n, const char* session,
                        const char* salt, int reserve, tgohip_lease** out);
int tgohip_lease_blocks(tgohip_lease* l, int32_t* out, int cap);
int tgohip_lease_reused(tgohip_lease* l);
int tgohip_lease_len(tgohip_lease* l);
int tgohip_lease_grow(tgohip_lease* l, int n);
int tgohip_lease_commit(tgohip_lease* l, const int32_t* ids, int n);
int tgohip_lease_publish(tgohip_lease* l, int written);
void tgohip_lease_release(tgohip_lease* l);
void tgohip_lease_free(tgohip_lease* l);

/* Scheduler (scheduler.go:34-397) driving tgohip_step: NewScheduler, Admit,
 * Step, Feed, Finish, Evict. The step's logits stay on the device; Step
 * reports per produced slot the greedy token (argmax) and whether it is
 * sampleable (Produced.Done). */
typedef struct tgohip_sched tgohip_sched;
/* slots n, chunk (0 = DefaultChunk 512, schedule.go:21), reserve (> 0),
 * max_rows per step. Requires tgohip_kv_alloc. */
tgohip_sched* tgohip_sched_new(tgohip_ctx* ctx, int n, int chunk, int reserve, int max_rows);
void tgohip_sched_free(tgohip_sched* s);
int tgohip_sched_admit(tgohip_sched* s, const int32_t* prompt, int n, int reserve);
int tgohip_sched_finish(tgohip_sched* s, int slot);
int tgohip_sched_evict(tgohip_sched* s);
int tgohip_sched_feed(tgohip_sched* s, int slot, int token);
int tgohip_sched_length(tgohip_sched* s, int slot);
/* One step. out arrays sized n: slot, token (greedy), done(0/1). Returns
 * the count produced; prefill_tokens/decodes as StepResult reports them. */
int tgohip_sched_step(tgohip_sched* s, int32_t* out_slot, int32_t* out_token,
                      int32_t* out_done, int32_t* prefill_tokens, int32_t* decodes,
                      tgohip_timings* t);

/* Admits a sequence whose prompt's KV is already resident (restored, or
 * synthetic in a benchmark): the slot starts decoding with token `feed`. The
 * prompt's whole blocks are published, as a prefill publishes them, so a later
 * prompt that begins with the same tokens shares those pages. */
int tgohip_sched_admit_prefilled(tgohip_sched* s, const int32_t* prompt, int n, int reserve,
                                 int feed);
int tgohip_sched_prefilling(tgohip_sched* s); /* live slots still mid-prefill */
int tgohip_sched_live(tgohip_sched* s);       /* live slots */
/* The ports of the last step (Batch.step's packing): sizes first with NULL
 * arrays, then the arrays (rows, rows*H, rows*H_kv, rows, B, B, B, B*max_pages).
 * In overlap mode, after the last step submitted has been collected (refused
 * while a step is in flight); posq/posk/slots are then derived on the host as
 * the device derived them. */
int tgohip_sched_last_step(tgohip_sched* s, int32_t* rows, int32_t* batch, int32_t* max_pages,
                           uint32_t* ids, uint32_t* posq, uint32_t* posk, uint32_t* slots,
                           uint32_t* lengths, uint32_t* extents, uint32_t* last,
                           uint32_t* pages);

/* Overlap mode (no counterpart in tgo, whose Batch.step packs, submits, waits
 * and reads back under the model's lock, batch.go:381-437; it is the host /
 * device overlap the path's next steps ask for). tgohip_sched_submit enqueues
 * the next step and returns without waiting; tgohip_sched_collect waits for
 * the oldest step in flight, commits it and reports its tokens. At most two
 * steps are in flight, so the host schedules step k+1 while the device runs
 * step k. A decode row's token is the previous step's argmax, read on the
 * device, and posq/posk/slots are derived on the device (tgohip_step with
 * NULL ports). The scheduler feeds every generated token itself:
 * tgohip_sched_feed refuses a slot it feeds. tgohip_sched_finish of a slot
 * with rows in flight takes effect for later submits at once and releases
 * its pages when those rows land. tgohip_sched_prefilling counts as if the
 * steps in flight had landed. Steps, and the tokens they produce, are those of
 * tgohip_sched_step when the caller admits and finishes the same sequences
 * before each submit as it would before each step. The context's argmax
 * buffer belongs to the scheduler between submits. */
int tgohip_sched_set_overlap(tgohip_sched* s, int on);
/* out arrays sized n: slot and done (0/1) per producing slot, in the order
 * collect reports them. Returns the count (0: nothing to step). */
int tgohip_sched_submit(tgohip_sched* s, int32_t* out_slot, int32_t* out_done,
                        int32_t* prefill_tokens, int32_t* decodes);
/* out arrays sized n: slot, token (greedy), done, as tgohip_sched_step
 * reports them. Returns the count (0: nothing in flight). */
int tgohip_sched_collect(tgohip_sched* s, int32_t* out_slot, int32_t* out_token,
                         int32_t* out_done, tgohip_timings* t);

/* ---- measurement ------------------------------------------------------- */
/* Brackets the attention launches of tgohip_step with HIP events on the
 * context's stream and accumulates their duration and algorithmic bytes
 * (every cached position a claimed row reads, K and V of all kv heads, once;
 * plus q read and the output written). on = 0: off; on = k >= 1: the launch
 * of every k-th layer (every layer's attention does the same work in a step;
 * each event record leaves the device idle a few microseconds). Turning it on
 * resets the sums. */
int tgohip_set_profile(tgohip_ctx* ctx, int on);
int tgohip_profile_read(tgohip_ctx* ctx, double* attn_ms, double* attn_bytes,
                        int64_t* launches);

/* The same for any of the step's kernels (measurement helper, no counterpart in
 * the reference; bench/bench.go:60-74 times whole steps only): mask has bit
 * TGOHIP_PROF_<kind> set for each kind timed, in every stride-th layer (the LM
 * head once per step). Reading a kind gives its summed duration, algorithmic
 * bytes (weights once, activations in and out; attention as above) and flops
 * (2*M*K*N; attention 4*d_h*H per visible query-key pair) over its launches. */
enum {
  TGOHIP_PROF_ATTN = 0,
  TGOHIP_PROF_QKV = 1,
  TGOHIP_PROF_O = 2,
  TGOHIP_PROF_GATEUP = 3,
  TGOHIP_PROF_DOWN = 4,
  TGOHIP_PROF_LMHEAD = 5,
  TGOHIP_PROF_KINDS = 6
};
int tgohip_set_profile_kernels(tgohip_ctx* ctx, int stride, int mask);
int tgohip_profile_read_kernel(tgohip_ctx* ctx, int kind, double* ms, double* bytes,
                               double* flops, int64_t* launches);
/* What this box reaches (measurement helper, no counterpart in the reference;
 * the benchmark reports it beside the published peaks): a streaming read of
 * read_bytes (16-byte non-temporal loads, grid-stride; a buffer the call allocates, fills
 * and frees) and a dense f16 MFMA loop (independent v_mfma_f32_32x32x16_f16
 * chains, four waves per workgroup, four workgroups per CU); medians of reps
 * timed launches on the context's stream. */
int tgohip_probe_peaks(tgohip_ctx* ctx, size_t read_bytes, int reps, double* read_gbps,
                       double* mfma_tflops);
/* Fills positions [0, positions) of every layer's K and V with seeded f16
 * N(0,1)*sigma: the context of sequences admitted already prefilled. */
int tgohip_kv_synth(tgohip_ctx* ctx, uint64_t seed, double sigma, int positions);

/* ---- weight conversion at load: weights/convert.go ---------------------- */
/* f32ToF16Bits over an array (weights/convert.go:133-180): RNE, saturate to
 * +-65504 (counted), flush below 2^-14 keeping sign, NaN -> 0x7e00. */
size_t tgohip_to_f16(const float* src, uint16_t* dst, size_t n);
/* int8 quantizer, one f16 scale per 32 flattened elements (convert.go:206-217). */
void tgohip_quantize_int8(const float* src, size_t n, int8_t* q, uint16_t* scales);
/* int4 asymmetric quantizer in the I4_TGO layout (weights/weights.go:694-743). */
void tgohip_quantize_int4(const float* src, size_t n, uint32_t* codes, uint16_t* scales,
                          uint16_t* zeros);

/* ---- checkpoint loading: safetensors/, weights/weights.go, model/qwen3.go -- */
typedef struct tgohip_st tgohip_st;
typedef struct tgohip_repo tgohip_repo;
/* Opens one safetensors file and validates its header as hostile input, as
 * safetensors.Open does (safetensors/safetensors.go:116-277): the length
 * prefix fits the file and a 100 MiB cap; the header is a JSON object; every
 * entry has a known dtype, two data_offsets inside the data region, no
 * negative dimension, an element count that does not overflow and that
 * matches the byte span; no two tensors share a byte; __metadata__ is a map
 * of strings. Entries are validated and kept in name order. NULL on refusal;
 * tgohip_last_error() names the tensor in the reference's words. */
tgohip_st* tgohip_st_open(const char* path);
void tgohip_st_close(tgohip_st* f);
int tgohip_st_count(const tgohip_st* f);
/* Entry i in name order (File.Names/Entry, safetensors.go:283-301): the name
 * and dtype strings live as long as f; up to 8 dimensions; the byte span is
 * relative to the end of the header. */
int tgohip_st_entry(const tgohip_st* f, int i, const char** name, const char** dtype, int* rank,
                    int64_t* shape, int64_t* begin, int64_t* end);
/* A tensor's raw bytes (File.Bytes, safetensors.go:302-323); returns the count. */
int64_t tgohip_st_read(const tgohip_st* f, const char* name, void* dst, int64_t cap);
/* Lowers the header cap (0 restores 100 MiB); the reference's tests lower it
 * the same way (safetensors_test.go:283-292). */
void tgohip_st_set_max_header(int64_t bytes);
/* A model directory (safetensors.OpenRepo, safetensors/repo.go:48-196): one
 * model.safetensors, or the shards model.safetensors.index.json names, checked
 * both ways (every indexed tensor is in its shard, every shard tensor is
 * indexed to it); shard names are plain file names; a config.json, when
 * present, is valid JSON. */
tgohip_repo* tgohip_repo_open(const char* dir);
void tgohip_repo_close(tgohip_repo* r);
int tgohip_repo_has(const tgohip_repo* r, const char* name);
/* The f32 plane of a tensor after the loader's conversions (convertOne,
 * weights/weights.go:552-627; convert.go:41-131): BF16 widened by a 16-bit
 * shift, F16 exactly, F32 as stored (other dtypes refused); [rows, cols]
 * transposed to [cols, rows] when transpose; then, when head_dim > 0, each
 * head_dim segment of the last axis re-paired y[2i] = x[i],
 * y[2i+1] = x[i + head_dim/2]. n is the element count of out. */
int tgohip_repo_plane(const tgohip_repo* r, const char* name, int transpose, int head_dim,
                      float* out, int64_t n);
/* weights.Load for a configured Qwen3 context (model/qwen3.go:54-205;
 * weights/weights.go:378-627): every port of the weight map, each tensor
 * present with the shape the config declares before any is converted, then
 * one at a time: plane as above (q/k projections and q/k-norm gains permuted,
 * projections and the head transposed), then form F16 (saturation over 1e-5
 * of a tensor refused), I8 or I4_TGO, uploaded through tgohip_weight /
 * tgohip_gain. The gathered embedding is capped at I8 under int4. tie: the
 * config's tie_word_embeddings -- the head is then the embedding tensor
 * transposed, and a checkpoint that also ships lm_head.weight is refused.
 * saturated (optional) receives the f16 saturation count. */
int tgohip_load_qwen3(tgohip_ctx* ctx, const tgohip_repo* r, int form, int tie, int64_t* saturated);

#ifdef __cplusplus
}
#endif
#endif
