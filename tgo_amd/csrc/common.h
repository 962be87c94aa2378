// common.h -- shared definitions for libtgohip (HIP/CDNA4, gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string>
#include <vector>

#include "../../include/tgohip.h"

namespace tgohip {

// Thread-local last error; every entry point that fails sets it.
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
std::string hip_message(hipError_t e, const char* what);

#define TGOHIP_HIP(call)                                                    \
  do {                                                                      \
    hipError_t _e = (call);                                                 \
    if (_e != hipSuccess) return ::tgohip::fail(TGOHIP_EDEVICE, ::tgohip::hip_message(_e, #call)); \
  } while (0)

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

// ---- attention plan (built on the host from lengths/extents) ----------
// One work item: a (sequence, kv head) pair's rows [tok0, tok0+ntok) of the
// sequence's extent against positions [kv_lo, kv_hi).
struct AttnItem {
  int32_t seq;
  int32_t kvh;
  int32_t tok0;
  int32_t ntok;
  int32_t kv_lo;
  int32_t kv_hi;
  int32_t part;  // partial slot for a split item, -1 when the item writes `out`
  int32_t mode;  // 0: rows <= 16, the four waves split the positions; 1: waves split rows;
                 // 2: an empty slot of the launch order; 3: a shared prefix: rows are
                 // the decode tokens of sequences seqlist[tok0 .. tok0+ntok) (G rows
                 // each), pages those of `seq`, every position visible. Mode 0 with
                 // kAttnSharedPages set: the item's positions include pages another
                 // sequence also reads (ordinary loads, not non-temporal ones).
};
constexpr int kAttnModeMask = 15;
constexpr int kAttnSharedPages = 16;
// One combine item: merges the partial results of a (sequence, kv head,
// tokens): first xparts parts of a shared prefix (the sequence's rows sit at
// row xrow of those parts), then nparts parts of its own positions.
struct AttnCombine {
  int32_t seq;
  int32_t kvh;
  int32_t tok0;
  int32_t ntok;
  int32_t part0;
  int32_t nparts;
  int32_t xpart0;  // first shared-prefix part, -1 when none
  int32_t xparts;
  int32_t xrow;
  int32_t pad;
};

constexpr int kAttnTile = 64;     // positions staged in LDS per iteration
constexpr int kAttnSplitDecode = 2560;   // positions per part of a split decode-style item
constexpr int kAttnSplitPrefill = 2048;  // positions per part of a split prefill-style item
constexpr int kAttnSplitShared = 512;    // positions per part of a shared-prefix item
constexpr int kAttnRowsP = 128;   // rows per prefill-style item (4 waves x 32)
constexpr int kHeadDim = 128;

struct AttnPlan {
  std::vector<AttnItem> items;
  std::vector<AttnCombine> combines;
  std::vector<int32_t> seqlist;  // sequences of shared-prefix items
  int64_t shared_positions = 0;  // positions read once for a group instead of per sequence
  std::vector<int32_t> cu;  // [B] flat row offset of each sequence
  int parts = 0;
  int claimed = 0;          // sum of extents
};


// ---- GEMM (kernels/gemm.hip) --------------------------------------------
// EPI_SWIGLU_X2 stores the SwiGLU output as an activation pair (below).
// EPI_QKROPE (the exact pipelined kernel, unsplit, derived rows): the QKV
// projection's q/k-norm, RoPE and K/V write run in its epilogue, as
// qk_rope_kv_kernel would run them on its output (qk_head_row below).
enum { EPI_F32 = 0, EPI_F16 = 1, EPI_RESID = 2, EPI_SWIGLU_F16 = 3, EPI_SWIGLU_F32 = 4,
       EPI_SWIGLU_X2 = 5, EPI_QKROPE = 6 };
// How an activation [M][K] is stored for a projection:
//   XK_F16  f16, rounded once (the fast f16 path, precision mode 0);
//   XK_F32  f32 (tgo's arithmetic; split into f16 hi + lo inside the kernel);
//   XK_X2   tgo's f32 activation already split by its producer: the f16 hi
//           plane [M][K] followed by the lo plane [M][K] (lo = f16(x - hi)),
//           so hi + lo carries ~22 bits of x. Same bytes as f32.
enum { XK_F16 = 0, XK_F32 = 1, XK_X2 = 2 };
// Output forms of the per-row producers (rmsnorm, attention): 0 f32, 1 f16,
// 2 the hi/lo pair of XK_X2 (lo plane `rows * width` elements after hi).
enum { OUT_F32 = 0, OUT_F16 = 1, OUT_X2 = 2 };

// A weight in the fragment-major device layout (see kernels/gemm.hip).
struct PackedWeight {
  int form = -1, K = 0, N = 0;
  void* wp = nullptr;
  half_t* ws = nullptr;
  half_t* wz = nullptr;
};

size_t packed_payload_bytes(int form, int K, int N);
size_t packed_scale_halves(int form, int K, int N);
// Repacks a canonical weight (device memory) into w. The sub-weight's n-block
// nb lands at n-block nb*nb_stride + nb_off of w (fused QKV / gate-up).
int repack_enqueue(int form, const void* plane, const uint16_t* scales, const uint16_t* zeros,
                   int K, int N, PackedWeight& w, int nb_stride, int nb_off, hipStream_t st);
int dequant_enqueue(const PackedWeight& w, void* out, bool f16out, hipStream_t st);
// Split-K workspace of a call: xk < 0 bounds every activation type and
// epilogue; an XK_* value gives exactly what an f32/f16-epilogue call over
// that activation type uses.
size_t gemm_workspace_bytes(const PackedWeight& w, int M, int ncu, int xk = -1);
// With defer != nullptr a split-K launch leaves its partial planes in the
// workspace ([splits][M][N] f32) and sets *defer = splits instead of running
// the reduction; the caller folds them into the consumer (rmsnorm,
// qk_rope_kv). *defer = 0 when the epilogue ran as usual.
int gemm_enqueue(const PackedWeight& w, const void* x, int xk, int M, void* y, int epi,
                 float* workspace, size_t ws_bytes, int ncu, hipStream_t st, int* defer = nullptr);

// ---- attention (kernels/attention.hip) -----------------------------------
struct AttnDevPlan {
  const AttnItem* items;
  const AttnCombine* combines;
  const int32_t* seqlist;
  const int32_t* cu;
  const uint32_t* lengths;
  const uint32_t* extents;
  const uint32_t* pages;
  float* part_o;
  float* part_ml;
};
int attn_build_plan(int T, int B, const uint32_t* lengths, const uint32_t* extents,
                    const uint32_t* pages, int max_pages, int block, int capacity, int H,
                    int Hkv, AttnPlan& plan, int cascade_min = 0, bool f32_q = false);
// out_form: OUT_F32, OUT_F16 or OUT_X2 (lo plane T * H * 128 elements after hi).
int attn_enqueue(const AttnPlan& plan, const AttnDevPlan& dp, const void* q, int q_f16,
                 const void* k, const void* v, void* out, int out_form, int T, int H, int Hkv,
                 int max_pages, int block, float scale, hipStream_t stream);

// ---- per-row kernels (kernels/elementwise.hip) ---------------------------
// Elements between consecutive split-K partial planes of an [M, N] f32
// product: M*N rounded up to whole 2 MiB pages, so each plane starts on a page.
inline size_t split_plane_stride(int M, int N) {
  const size_t e = (size_t)M * N, page = ((size_t)2 << 20) / sizeof(float);
  return (e + page - 1) / page * page;
}

struct QKRopeArgs {
  const float* qkv;       // [T, (H + 2*Hkv) * 128], or nsplit partial planes of it
  int nsplit;             // 0: qkv is the projection; > 0: sum the planes (split order)
  size_t plane;           // elements per partial plane
  const float* qnorm;     // [128]
  const float* knorm;     // [128]
  const uint32_t* posq;   // [T*H], or null: rowpos holds the row's position
  const uint32_t* posk;   // [T*Hkv]
  const uint32_t* slots;  // [T]
  const uint32_t* rowpos; // [T] (derive_rows_kernel) when posq is null
  const double* inv_freq; // [64]: base^(-2i/128), computed once on the host in double
  void* q;                // [T, H, 128], f32 or (q_f16) f16
  half_t* kc;             // layer view [C, Hkv, 128]
  half_t* vc;
  int H, Hkv, capacity;
  float eps;
  int q_f16;
  const float4_t* rope;   // [T][32] (rope_table), or null: the kernel computes the angles
};

// Sum over the 32 lanes of a half wave (lanes 0-31 and 32-63 separately).
__device__ __forceinline__ float qk_half_wave_sum(float v) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// One head row hh of row t (nn/attention.go:192-232), the lane's dims
// 4*l32 .. 4*l32+3 of it in v: a value head is narrowed and scattered to
// slot; a q or k head is RMS-normalized over its 128 dims (the half wave
// sums the squares), scaled by its gain, rotated in interleaved pairs by
// (c0, s0) and (c1, s1), and stored (q to a.q, k narrowed to slot). A slot at
// or past capacity writes nothing. angles(pos) gives (c0, s0, c1, s1) for the
// head's position, called only for q and k heads. qk_rope_kv_kernel and the
// QKV projection's fused epilogue both call this, so both compute the same
// values from the same projection output.
template <typename Angles>
__device__ __forceinline__ void qk_head_row(const QKRopeArgs& a, int t, int hh, int l32, float4_t v,
                                            uint32_t slot, Angles angles) {
  const bool write = slot < (uint32_t)a.capacity;
  if (hh >= a.H + a.Hkv) {
    if (write) {
      const int vh = hh - a.H - a.Hkv;
      const half4_t hv = {(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
      *(half4_t*)(a.vc + ((size_t)slot * a.Hkv + vh) * kHeadDim + 4 * l32) = hv;
    }
    return;
  }
  const bool isq = hh < a.H;
  const float* gain = isq ? a.qnorm : a.knorm;
  // The fused multiply-adds are written out (in the order the compiler chose
  // for qk_rope_kv_kernel when it contracted the expressions itself), so
  // every kernel that inlines this computes the same bits: left to
  // contraction, x0 s0 + x1 c0 became fma(x1, c0, x0 s0) in one kernel and
  // fma(s0, x0, x1 c0) in another.
  const float ss = qk_half_wave_sum(
      __builtin_fmaf(v[3], v[3], __builtin_fmaf(v[2], v[2], __builtin_fmaf(v[0], v[0], v[1] * v[1]))));
  const float sc = 1.0f / sqrtf(ss / (float)kHeadDim + a.eps);
  const float4_t g = *(const float4_t*)(gain + 4 * l32);
  const float x0 = v[0] * sc * g[0], x1 = v[1] * sc * g[1];
  const float x2 = v[2] * sc * g[2], x3 = v[3] * sc * g[3];
  float c0, s0, c1, s1;
  angles(isq, hh, c0, s0, c1, s1);
  const float y0 = __builtin_fmaf(x0, c0, -(x1 * s0)), y1 = __builtin_fmaf(x1, c0, x0 * s0);
  const float y2 = __builtin_fmaf(x2, c1, -(x3 * s1)), y3 = __builtin_fmaf(x3, c1, x2 * s1);
  if (isq && a.q_f16) {
    const half4_t hq = {(half_t)y0, (half_t)y1, (half_t)y2, (half_t)y3};
    *(half4_t*)((half_t*)a.q + ((size_t)t * a.H + hh) * kHeadDim + 4 * l32) = hq;
  } else if (isq) {
    *(float4_t*)((float*)a.q + ((size_t)t * a.H + hh) * kHeadDim + 4 * l32) = float4_t{y0, y1, y2, y3};
  } else if (write) {
    const int kh = hh - a.H;
    const half4_t hk = {(half_t)y0, (half_t)y1, (half_t)y2, (half_t)y3};
    *(half4_t*)(a.kc + ((size_t)slot * a.Hkv + kh) * kHeadDim + 4 * l32) = hk;
  }
}

// The QKV projection of an activation pair [M][K] with qk_head_row in its
// epilogue (EPI_QKROPE) instead of an f32 output for qk_rope_kv_kernel: when
// gemm_qkrope_fusable, gemm_enqueue_qkrope does both in one launch (qa as
// for qk_rope_kv_kernel, with rope set; qkv and the split fields unused).
bool gemm_qkrope_fusable(const PackedWeight& w, int M, int ncu);
int gemm_enqueue_qkrope(const PackedWeight& w, const void* x, int M, const QKRopeArgs& qa, int ncu,
                        hipStream_t st);
// ids[t] with bit 31 set names a member b = ids[t] & 0x7fffffff whose token is
// feed[b] (the previous step's argmax, left on the device).
void launch_embed(const uint32_t* ids, int T, const void* table, const uint16_t* scales, int form,
                  int d, float* h, hipStream_t st, const int32_t* feed = nullptr);
// out_form: OUT_F32, OUT_F16 or OUT_X2 (lo plane nrows * w elements after hi).
void launch_rmsnorm(float* x, const uint32_t* rows, int nrows, const float* g, int w,
                    float eps, void* out, int out_form, hipStream_t st, const float* part = nullptr,
                    int nsplit = 0, size_t plane = 0);
void launch_qk_rope_kv(const QKRopeArgs& a, int T, hipStream_t st);
// posq/posk/slots derived on the device from the members (NewBatchStep's
// values): row cu[b] + j of member b sits at lengths[b] - extents[b] + j; rows
// past `total` repeat member pad's last position with slot = capacity.
struct DeriveArgs {
  const int32_t* cu;
  const uint32_t* lengths;
  const uint32_t* extents;
  const uint32_t* pages;
  int B, max_pages, block, total, pad, T, capacity;
  uint32_t* pos;   // [T]
  uint32_t* slot;  // [T]
};
void launch_derive_rows(const DeriveArgs& a, hipStream_t st);
// table[t * 32 + l] = {cos, sin} of rowpos[t] at the rotary frequencies 2l and
// 2l + 1 (inv_freq), computed as qk_rope_kv_kernel would: once per step for
// every layer.
void launch_rope_table(const uint32_t* rowpos, int T, const double* inv_freq, float4_t* table,
                       hipStream_t st);
// keep_idle: members with extent 0 leave out[b] as it is (else out[b] = -1);
// extents == null: every row is live. margin (nullable): the row's top-two
// margin in float64 (TopTwoMargin). zero_idle: the logits rows of members with
// extent 0 are zeroed first. scratch: argmax_scratch_bytes(B, V) of device
// memory for the per-chunk partials (a size that also serves any call with
// fewer rows).
size_t argmax_scratch_bytes(int B, int V);
// cidx != null: the logits hold `rows` compacted rows, those of the members
// that worked; member b's is row cidx[b] (-1: extent 0, token -1 unless
// keep_idle, margin 0). extents and zero_idle then play no part.
void launch_argmax(float* logits, int B, int V, const uint32_t* extents, int32_t* out,
                   void* scratch, hipStream_t st, int keep_idle = 0, double* margin = nullptr,
                   int zero_idle = 0, int rows = 0, const int32_t* cidx = nullptr);
void launch_synth_f16(uint64_t seed, uint64_t stream, size_t n, double sigma, uint16_t* out,
                      hipStream_t st);
void launch_synth_absf16(uint64_t seed, uint64_t stream, size_t n, double sigma, uint16_t* out,
                         hipStream_t st);
void launch_synth_i4sym(uint64_t seed, uint64_t stream, int K, int N, uint32_t* out, hipStream_t st);
void launch_synth_i4tgo(uint64_t seed, uint64_t stream, size_t n, uint32_t* out, hipStream_t st);
void launch_synth_zero(uint64_t seed, uint64_t stream, size_t n, uint16_t* out, hipStream_t st);
void launch_synth_i8(uint64_t seed, uint64_t stream, size_t n, int8_t* out, hipStream_t st);
// load-time quantizers (the host's tgohip_quantize_int8 / _int4, bit for bit)
void launch_quantize_i8(const float* w, size_t n, int8_t* q, uint16_t* scales, hipStream_t st);
void launch_quantize_i4tgo(const float* w, size_t n, uint32_t* codes, uint16_t* scales,
                           uint16_t* zeros, hipStream_t st);
void launch_synth_gain(uint64_t seed, uint64_t stream, size_t n, float* out, hipStream_t st);
void launch_fill_f32(float* p, size_t n, float v, hipStream_t st);

// ---- peak probes (kernels/probe.hip) ---------------------------------------
int probe_read_enqueue(const void* p, size_t bytes, uint32_t* sink, hipStream_t st);
double probe_mfma_enqueue(int blocks, int iters, float* sink, hipStream_t st);

}  // namespace tgohip
