// elementwise.hip -- the per-row kernels around the projections and attention
// of one step (model/qwen3_graph.go:32-128):
//   embed_kernel        GatherRows / QuantGatherRows of the embedding (:54-61)
//   rmsnorm_kernel      RMSNorm (nn/blocks.go:53-55) fused with the cast to the
//                       next projection's operand dtype, optionally gathering
//                       rows (the head's GatherRows(h, last), :117)
//   qk_rope_kv_kernel   q/k RMSNorm per head + interleaved RoPE + f16 narrowing +
//                       ScatterRows into the paged pool, slot >= capacity dropped
//                       (nn/attention.go:192-232, plan.go:182-192)
//   rope_table_kernel   the rows' rotary cos and sin (nn/attention.go:203-211),
//                       once per step for every layer's qk_rope_kv_kernel
//   argmax_*_kernel     greedy token, first strict maximum (sample/stages.go:196),
//                       and the top-two margin
//   synth_* kernels     seeded random-init weights, bit-identical to the CPU
//                       restatement's generator
#include "../common.h"

#include <algorithm>

namespace tgohip {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// h[t, :] = table[ids[t], :] (f16) or q * scale (int8, one scale per 32
// flattened elements). An id with bit 31 set is a member index whose token
// is feed[member].
__global__ void embed_kernel(const uint32_t* ids, const void* table, const uint16_t* scales,
                             int form, int d, float* h, const int32_t* feed) {
  const int t = blockIdx.x;
  const uint32_t id = ids[t];
  const uint32_t tok = (id >> 31) ? (uint32_t)feed[id & 0x7fffffffu] : id;
  const size_t base = (size_t)tok * d;
  for (int i = threadIdx.x; i < d; i += blockDim.x) {
    float v;
    if (form == TGOHIP_FORM_F16) {
      v = (float)((const half_t*)table)[base + i];
    } else {
      const size_t e = base + i;
      v = (float)((const int8_t*)table)[e] * (float)(*(const half_t*)&scales[e / 32]);
    }
    h[(size_t)t * d + i] = v;
  }
}

// out[r, :] = x[src(r), :] * rsqrt(mean(x^2) + eps) * g, stored f16 or f32.
// src(r) = rows ? rows[r] : r. One block per row, a float4 per thread (up to
// 1024 threads; wider rows loop): every load of a row is in flight at once.
// With nsplit > 0 the residual add of a split-K projection is still pending:
// x[src, :] += sum_s part[s][src, :] (summed in split order, as
// gemm_reduce_kernel would) is done here first and written back to x. When
// gathering (rows != null: the head's last rows, which two members may share)
// the sum is used but x is left as it is.
// acc += the N planes at p, p + plane, ... (element offset off), added in
// plane order after all N loads are issued.
template <int N>
__device__ __forceinline__ void add_planes(float4_t& acc, const float* p, size_t plane, size_t off) {
  float4_t v[N];
#pragma unroll
  for (int u = 0; u < N; u++) v[u] = *(const float4_t*)(p + (size_t)u * plane + off);
#pragma unroll
  for (int u = 0; u < N; u++) acc += v[u];
}

// Sum of nsplit split-K partial planes at element offset off, in split order
// (the order gemm_reduce_kernel adds them). Up to eight planes' loads are in
// flight together; a loop of load-then-add waited for each in turn (8 round
// trips for the 8-split projections of a 128-row step).
__device__ __forceinline__ float4_t sum_planes(const float* part, int nsplit, size_t plane,
                                               size_t off) {
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < nsplit; s0 += 8) {
    const float* p = part + (size_t)s0 * plane;
    switch (min(nsplit - s0, 8)) {
      case 1: add_planes<1>(acc, p, plane, off); break;
      case 2: add_planes<2>(acc, p, plane, off); break;
      case 3: add_planes<3>(acc, p, plane, off); break;
      case 4: add_planes<4>(acc, p, plane, off); break;
      case 5: add_planes<5>(acc, p, plane, off); break;
      case 6: add_planes<6>(acc, p, plane, off); break;
      case 7: add_planes<7>(acc, p, plane, off); break;
      default: add_planes<8>(acc, p, plane, off); break;
    }
  }
  return acc;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; i++) t += red[i];
  return t;
}

// R > 0: every thread owns at most R float4s of the row (w <= 4 R blockDim.x)
// and keeps them in registers between the sum of squares and the scaling;
// R = 0: any width, the second pass reloads the row.
// out_form OUT_X2: the f32 result as its f16 hi plane [nrows][w] and lo plane
// (f16(x - hi)) right after it, the activation pair the exact projections read.
template <int R>
__global__ __launch_bounds__(1024) void rmsnorm_kernel(float* x, const uint32_t* rows,
                                                       const float* g, int w, float eps,
                                                       void* out, int out_form, const float* part,
                                                       int nsplit, size_t plane) {
  __shared__ float red[16];
  const int r = blockIdx.x;
  const int step = blockDim.x * 4;
  const size_t src = (size_t)(rows ? rows[r] : (uint32_t)r) * w;
  auto finish = [&](const float4_t& v, int i, float sc) {
    const float4_t gg = *(const float4_t*)(g + i);
    float4_t o;
#pragma unroll
    for (int j = 0; j < 4; j++) o[j] = v[j] * sc * gg[j];
    if (out_form == OUT_F32) {
      *(float4_t*)((float*)out + (size_t)r * w + i) = o;
    } else {
      half4_t hv = {(half_t)o[0], (half_t)o[1], (half_t)o[2], (half_t)o[3]};
      *(half4_t*)((half_t*)out + (size_t)r * w + i) = hv;
      if (out_form == OUT_X2) {
        half4_t lv;
#pragma unroll
        for (int j = 0; j < 4; j++) lv[j] = (half_t)(o[j] - (float)hv[j]);
        *(half4_t*)((half_t*)out + (size_t)gridDim.x * w + (size_t)r * w + i) = lv;
      }
    }
  };
  float ss = 0.f;
  if constexpr (R > 0) {
    float4_t v[R];
#pragma unroll
    for (int u = 0; u < R; u++) {
      const int i = threadIdx.x * 4 + u * step;
      if (i >= w) break;
      v[u] = *(const float4_t*)(x + src + i);
      if (nsplit > 0) {
        v[u] += sum_planes(part, nsplit, plane, src + i);
        if (!rows) *(float4_t*)(x + src + i) = v[u];
      }
      ss += v[u][0] * v[u][0] + v[u][1] * v[u][1] + v[u][2] * v[u][2] + v[u][3] * v[u][3];
    }
    ss = block_sum(ss, red);
    const float sc = 1.0f / sqrtf(ss / (float)w + eps);
#pragma unroll
    for (int u = 0; u < R; u++) {
      const int i = threadIdx.x * 4 + u * step;
      if (i >= w) break;
      finish(v[u], i, sc);
    }
  } else {
    for (int i = threadIdx.x * 4; i < w; i += step) {
      float4_t v = *(const float4_t*)(x + src + i);
      if (nsplit > 0) {
        v += sum_planes(part, nsplit, plane, src + i);
        if (!rows) *(float4_t*)(x + src + i) = v;
      }
      ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
    }
    ss = block_sum(ss, red);
    const float sc = 1.0f / sqrtf(ss / (float)w + eps);
    for (int i = threadIdx.x * 4; i < w; i += step) {
      float4_t v = *(const float4_t*)(x + src + i);
      if (nsplit > 0 && rows) v += sum_planes(part, nsplit, plane, src + i);
      finish(v, i, sc);
    }
  }
}


// The rows' positions and cache slots, as model.NewBatchStep packs them
// (batch.go:310-340): block b < B writes member b's rows cu[b] + j at position
// lengths[b] - extents[b] + j, slot pages[b][p / block] * block + p % block;
// block B writes the padding rows past `total`: member pad's last position,
// slot = capacity (a dropped write).
__global__ __launch_bounds__(256) void derive_rows_kernel(DeriveArgs a) {
  const int b = blockIdx.x;
  if (b < a.B) {
    const int n = (int)a.extents[b];
    const int first = (int)a.lengths[b] - n, t0 = a.cu[b];
    const uint32_t* prow = a.pages + (size_t)b * a.max_pages;
    for (int j = threadIdx.x; j < n; j += blockDim.x) {
      const int p = first + j;
      a.pos[t0 + j] = (uint32_t)p;
      a.slot[t0 + j] = prow[p / a.block] * (uint32_t)a.block + (uint32_t)(p % a.block);
    }
  } else {
    const uint32_t p = a.lengths[a.pad] - 1;
    for (int t = a.total + threadIdx.x; t < a.T; t += blockDim.x) {
      a.pos[t] = p;
      a.slot[t] = (uint32_t)a.capacity;
    }
  }
}

// One block (4 waves) per token. A wave takes two head rows at a time (lanes
// 0-31 head 2k, lanes 32-63 head 2k+1, wave w taking k = w, w+4, ...); a lane
// owns four consecutive dims, the rotated pairs (4l, 4l+1) and (4l+2, 4l+3),
// with 16-byte loads. (Loading a batch of a wave's rows before working on any
// measured 65% slower.)
__global__ __launch_bounds__(256) void qk_rope_kv_kernel(QKRopeArgs a) {
  const int t = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6 | blockIdx.y << 2;
  const int half = lane >> 5, l32 = lane & 31;
  const int NH = a.H + 2 * a.Hkv;
  const int W = NH * kHeadDim;
  const uint32_t slot = a.slots[t];
  const int dpos = a.rowpos ? (int)a.rowpos[t] : 0;  // the row's position when derived
  int cpos = -1;
  float c0 = 1.f, s0 = 0.f, c1 = 1.f, s1 = 0.f;
  const double inv0 = a.inv_freq[2 * l32], inv1 = a.inv_freq[2 * l32 + 1];
  if (a.rope) {
    // the row's angles, computed once per step (the f64 sin and cos per wave
    // were most of this kernel's time)
    const float4_t cs = a.rope[(size_t)t * 32 + l32];
    c0 = cs[0];
    s0 = cs[1];
    c1 = cs[2];
    s1 = cs[3];
    cpos = dpos;
  }
  for (int k = wave; 2 * k < NH; k += 4 * gridDim.y) {
    const int hh = 2 * k + half;
    if (hh >= NH) continue;  // an odd head count leaves the last half wave idle
    // split-K projection: the row is the sum of the partial planes, in split order
    const size_t off = (size_t)t * W + hh * kHeadDim + 4 * l32;
    float4_t v;
    if (a.nsplit == 0) {
      v = *(const float4_t*)(a.qkv + off);
    } else {
      v = sum_planes(a.qkv, a.nsplit, a.plane, off);
    }
    qk_head_row(a, t, hh, l32, v, slot, [&](bool isq, int h2, float& cc0, float& ss0, float& cc1,
                                             float& ss1) {
      const int pos = a.rowpos ? dpos
                      : isq   ? (int)a.posq[(size_t)t * a.H + h2]
                              : (int)a.posk[(size_t)t * a.Hkv + (h2 - a.H)];
      if (pos != cpos) {
        const double ang0 = (double)pos * inv0, ang1 = (double)pos * inv1;
        c0 = (float)cos(ang0);
        s0 = (float)sin(ang0);
        c1 = (float)cos(ang1);
        s1 = (float)sin(ang1);
        cpos = pos;
      }
      cc0 = c0;
      ss0 = s0;
      cc1 = c1;
      ss1 = s1;
    });
  }
}

// First index of the strict maximum of each row (sample/stages.go:196-206).
// Go's loop keeps best = x[0] and takes i only when x[i] > best: the first
// index of the maximum, NaN never taken after index 0, and 0 when x[0] is NaN
// or nothing exceeds it.
//
// With margin != null the same pass gives TopTwoMargin
// (internal/conformance/measure.go:91-110): the largest logit minus the
// second largest, counting a repeated maximum twice (margin 0), in float64.
// Go seeds (first, second) with x[0], x[1] and folds the rest with strict
// comparisons, so a NaN after index 1 is never taken; the order-free
// reduction here keeps the top two of the non-NaN values and restates Go's
// two seeded cases: x[0] NaN gives NaN, and x[1] NaN gives NaN unless a later
// value exceeds x[0] (exactly when the argmax is not 0).
//
// Two kernels. argmax_part_kernel: S workgroups per row, workgroup s scanning
// the s-th contiguous chunk (whole float4s when V % 4 == 0), each thread its
// elements in ascending order, leaving the chunk's (top1, top2, index of the
// first top1) in part[b * S + s]. One workgroup per row left the C4 head's
// 130 rows on half the CUs and VALU-bound (62 us for 79 MB). With zero_idle
// the rows of members that contributed nothing (extents[b] == 0) are zeroed
// instead of scanned. argmax_final_kernel: one thread per row merges its S
// chunks and applies Go's x[0] / x[1] rules.
struct Top2 {
  float t1, t2;  // largest and second largest non-NaN values (-inf when none)
  int i1;        // first index of t1 (0x7fffffff when none)
  int pad;
};

// Folds (b1, b2, bi) into (t1, t2, i1): equal maxima keep the smaller index.
__device__ __forceinline__ void top2_merge(float& t1, float& t2, int& i1, float b1, float b2,
                                           int bi) {
  if (b1 > t1 || (b1 == t1 && bi < i1)) i1 = bi;
  const float lo = fminf(t1, b1), hi2 = fmaxf(t2, b2);  // t1, b1 are never NaN
  t1 = fmaxf(t1, b1);
  t2 = fmaxf(lo, hi2);
}

// Per element: the strict comparisons of Go's loops, NaN false in both.
__device__ __forceinline__ void top2_take(float& t1, float& t2, int& i1, float v, int i) {
  const bool c1 = v > t1, c2 = v > t2;
  t2 = c1 ? t1 : (c2 ? v : t2);
  t1 = c1 ? v : t1;
  i1 = c1 ? i : i1;
}

constexpr int kArgmaxThreads = 256;

// Chunks per row: about 512 workgroups in all, at most 16, each chunk at
// least 4096 logits.
static inline int argmax_chunks(int B, int V) {
  int s = (512 + B - 1) / std::max(B, 1);
  s = std::min(s, std::max(1, V / 4096));
  return std::max(1, std::min(s, 16));
}

// B * argmax_chunks(B, V) <= B * ceil(512 / B) < 512 + B: enough for any
// call with at most B rows, whatever V.
size_t argmax_scratch_bytes(int B, int V) {
  (void)V;
  return (size_t)(512 + std::max(B, 0)) * sizeof(Top2);
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_part_kernel(float* logits, int V, int S,
                                                                     const uint32_t* extents,
                                                                     int zero_idle, Top2* part) {
  __shared__ float sv1[kArgmaxThreads / 64], sv2[kArgmaxThreads / 64];
  __shared__ int si[kArgmaxThreads / 64];
  const int b = blockIdx.x, s = blockIdx.y, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  float* row = logits + (size_t)b * V;
  const bool vec = (V & 3) == 0;  // rows 16-byte aligned: whole float4 chunks
  const int units = vec ? V / 4 : V;
  const int u0 = (int)((int64_t)units * s / S), u1 = (int)((int64_t)units * (s + 1) / S);
  float t1 = -INFINITY, t2 = -INFINITY;
  int i1 = 0x7fffffff;
  if (zero_idle && extents[b] == 0) {
    // an idle member's row: zeros (so the final pass gives 0 and margin 0)
    for (int u = u0 + t; u < u1; u += kArgmaxThreads) {
      if (vec) ((float4_t*)row)[u] = float4_t{0.f, 0.f, 0.f, 0.f};
      else row[u] = 0.f;
    }
    if (t == 0) part[(size_t)b * S + s] = Top2{0.f, u1 - u0 > 1 || vec ? 0.f : -INFINITY,
                                               vec ? 4 * u0 : u0, 0};
    return;
  }
  if (vec) {
    // Eight float4 loads in flight per thread; its elements still in ascending order.
    const float4_t* row4 = (const float4_t*)row;
    int u = u0 + t;
    for (; u + 7 * kArgmaxThreads < u1; u += 8 * kArgmaxThreads) {
      float4_t v[8];
#pragma unroll
      for (int k = 0; k < 8; k++) v[k] = row4[u + k * kArgmaxThreads];
#pragma unroll
      for (int k = 0; k < 8; k++)
#pragma unroll
        for (int j = 0; j < 4; j++) top2_take(t1, t2, i1, v[k][j], 4 * (u + k * kArgmaxThreads) + j);
    }
    for (; u < u1; u += kArgmaxThreads) {
      const float4_t v = row4[u];
#pragma unroll
      for (int j = 0; j < 4; j++) top2_take(t1, t2, i1, v[j], 4 * u + j);
    }
  } else {
    for (int u = u0 + t; u < u1; u += kArgmaxThreads) top2_take(t1, t2, i1, row[u], u);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float b1 = __shfl_xor(t1, o, 64), b2 = __shfl_xor(t2, o, 64);
    const int bi = __shfl_xor(i1, o, 64);
    top2_merge(t1, t2, i1, b1, b2, bi);
  }
  if (lane == 0) {
    sv1[wave] = t1;
    sv2[wave] = t2;
    si[wave] = i1;
  }
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < kArgmaxThreads / 64; w++) top2_merge(t1, t2, i1, sv1[w], sv2[w], si[w]);
    part[(size_t)b * S + s] = Top2{t1, t2, i1, 0};
  }
}

// extents == null treats every row as live. cidx != null: the logits hold
// only the members that worked, compacted; member b's row is cidx[b] (-1 for
// a member with extent 0: no token, margin 0, its logits row is not there).
__global__ void argmax_final_kernel(const float* logits, int B, int V, int S,
                                    const uint32_t* extents, const Top2* part, int32_t* out,
                                    int keep_idle, double* margin, const int32_t* cidx) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  int rowi = b;
  if (cidx) {
    rowi = cidx[b];
    if (rowi < 0) {
      if (!keep_idle) out[b] = -1;
      if (margin) margin[b] = 0.0;
      return;
    }
  }
  const Top2* p = part + (size_t)rowi * S;
  float t1 = p[0].t1, t2 = p[0].t2;
  int i1 = p[0].i1;
  for (int s = 1; s < S; s++) top2_merge(t1, t2, i1, p[s].t1, p[s].t2, p[s].i1);
  // x[0] itself, and NaN at x[0], are Go's starting point
  const float* row = logits + (size_t)rowi * V;
  const float x0 = row[0];
  int r = i1;
  if (x0 != x0 || i1 == 0x7fffffff || !(t1 > x0)) r = 0;
  const bool live = cidx || !extents || extents[b] != 0;
  if (live) out[b] = r;
  else if (!keep_idle) out[b] = -1;
  if (margin) {
    const float x1 = row[1];
    double mg = (double)t1 - (double)t2;
    if (x0 != x0 || (x1 != x1 && r == 0)) mg = __builtin_nan("");
    margin[b] = mg;
  }
}

// ---- seeded synthesis (the CPU restatement's generator, restated) ---------
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t hash3(uint64_t seed, uint64_t stream, uint64_t idx) {
  return splitmix64(splitmix64(seed * 0x100000001B3ull + stream) + idx);
}
__device__ __forceinline__ double normal_ih(uint64_t seed, uint64_t stream, uint64_t idx) {
  const uint64_t m = (1ull << 21) - 1;
  int64_t s = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint64_t h = hash3(seed, stream, idx * 4 + (uint64_t)j);
    s += (int64_t)(h & m) + (int64_t)((h >> 21) & m) + (int64_t)((h >> 42) & m);
  }
  return (double)(s - 6 * (int64_t)(1 << 21)) / (double)(1 << 21);
}

// f32ToF16Bits (weights/convert.go:153-180) on the device: NaN -> 0x7e00,
// saturate to +-65504, flush below 2^-14 keeping sign, else RNE.
__device__ __forceinline__ uint16_t f16_loader_bits(float x) {
  const uint32_t b = __float_as_uint(x);
  const uint16_t sign = (uint16_t)((b >> 16) & 0x8000);
  if ((b & 0x7fffffffu) > 0x7f800000u) return 0x7e00;
  const float a = __uint_as_float(b & 0x7fffffffu);
  if (a > 65504.0f) return sign | 0x7bff;
  if (a < 1.0f / 16384.0f) return sign;
  const int32_t e = (int32_t)((b >> 23) & 0xff) - 127;
  const uint32_t mant = b & 0x7fffffu;
  uint32_t keep = mant >> 13;
  const uint32_t rest = mant & 0x1fffu, half = 0x1000u;
  if (rest > half || (rest == half && (keep & 1))) keep++;
  return (uint16_t)(sign | (uint16_t)(((uint32_t)(e + 15) << 10) + keep));
}

// ---- load-time quantizers on the device ------------------------------------
// The host's tgohip_quantize_int8 (quantizeInto, weights/convert.go:206-217)
// and tgohip_quantize_int4 (the int4 triple of weights/weights.go:694-743)
// restated so that a checkpoint's f32 planes quantize where they are uploaded,
// with the same bits: the same f32 and f64 operations in the same order (IEEE
// division, round-half-even), the loader's f16 rule (f16_loader_bits), and
// std::min / std::max's comparisons, so a
// NaN is skipped or clamped exactly as on the host. One thread per group, its
// elements in order.
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(half_t, h);  // the rule's outputs: normal, zero, +-65504, NaN
}

__global__ void quantize_i8_kernel(const float* w, size_t n, int8_t* q, uint16_t* scales) {
  const size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x, lo = g * 32;
  if (lo >= n) return;
  const size_t hi = lo + 32 < n ? lo + 32 : n;
  float peak = 0.f;
  for (size_t i = lo; i < hi; i++) {
    const float a = fabsf(w[i]);
    peak = (peak < a) ? a : peak;  // std::max(peak, a)
  }
  const uint16_t s16 = f16_loader_bits(peak / 127.0f);
  const float s = f16_bits_to_f32(s16);
  scales[g] = s16;
  for (size_t i = lo; i < hi; i++) {
    double v = s > 0 ? rint((double)w[i] / (double)s) : 0.0;
    v = (v < 127.0) ? v : 127.0;    // std::min(127.0, v)
    v = (-127.0 < v) ? v : -127.0;  // std::max(-127.0, v)
    q[i] = (int8_t)v;
  }
}

__global__ void quantize_i4tgo_kernel(const float* w, size_t n, uint32_t* codes, uint16_t* scales,
                                      uint16_t* zeros) {
  const size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x, lo = g * 128;
  if (lo >= n) return;
  const size_t hi = lo + 128 < n ? lo + 128 : n;
  float mn = w[lo], mx = w[lo];
  for (size_t i = lo; i < hi; i++) {
    const float x = w[i];
    mn = (x < mn) ? x : mn;  // std::min(mn, x)
    mx = (mx < x) ? x : mx;  // std::max(mx, x)
  }
  const float sr = (mx - mn) / 15.0f;
  uint16_t s16 = f16_loader_bits(sr > 0 ? sr : 1.0f);
  float s = f16_bits_to_f32(s16);
  if (s == 0) {
    s16 = 0x3c00;
    s = 1.0f;
  }
  double zf = rint(-(double)mn / (double)s);
  zf = (zf < 15.0) ? zf : 15.0;  // std::min(15.0, zf)
  zf = (0.0 < zf) ? zf : 0.0;    // std::max(0.0, zf)
  scales[g] = s16;
  zeros[g] = f16_loader_bits((float)zf);
  for (size_t i0 = lo; i0 < hi; i0 += 8) {
    uint32_t word = 0;
    for (size_t i = i0; i < i0 + 8 && i < hi; i++) {
      double v = rint((double)w[i] / (double)s + zf);
      v = (v < 15.0) ? v : 15.0;
      v = (0.0 < v) ? v : 0.0;
      word |= ((uint32_t)v & 15u) << (4 * (i % 8));
    }
    codes[i0 / 8] = word;
  }
}

void launch_quantize_i8(const float* w, size_t n, int8_t* q, uint16_t* scales, hipStream_t st) {
  const size_t groups = (n + 31) / 32;
  hipLaunchKernelGGL(quantize_i8_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st, w, n,
                     q, scales);
}
void launch_quantize_i4tgo(const float* w, size_t n, uint32_t* codes, uint16_t* scales,
                           uint16_t* zeros, hipStream_t st) {
  const size_t groups = (n + 127) / 128;
  hipLaunchKernelGGL(quantize_i4tgo_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st,
                     w, n, codes, scales, zeros);
}

// F16 plane: loader-rule f16 of f32(N(0,1) * sigma).
__global__ void synth_f16_kernel(uint64_t seed, uint64_t stream, size_t n, double sigma,
                                 uint16_t* out) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = f16_loader_bits((float)(normal_ih(seed, stream, i) * sigma));
}
// |N(0,1)| * sigma as loader-rule f16 (scales).
__global__ void synth_absf16_kernel(uint64_t seed, uint64_t stream, size_t n, double sigma,
                                    uint16_t* out) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = f16_loader_bits((float)(fabs(normal_ih(seed, stream, i)) * sigma));
}
// I4_SYM codes: word (r, n) of [K/8][N], k = 8r+i -> nibble hash&15.
__global__ void synth_i4sym_kernel(uint64_t seed, uint64_t stream, int K, int N, uint32_t* out) {
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (size_t)(K / 8) * N) return;
  const size_t r = t / N, n = t % N;
  uint32_t w = 0;
  for (int i = 0; i < 8; i++) {
    const uint64_t e = (uint64_t)(r * 8 + i) * (uint64_t)N + n;
    w |= (uint32_t)(hash3(seed, stream, e) & 15u) << (4 * i);
  }
  out[t] = w;
}
// I4_TGO codes over the flattened plane: element e -> hash&15.
__global__ void synth_i4tgo_kernel(uint64_t seed, uint64_t stream, size_t n, uint32_t* out) {
  const size_t wi = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (wi >= (n + 7) / 8) return;
  uint32_t w = 0;
  for (int i = 0; i < 8; i++) {
    const size_t e = wi * 8 + i;
    if (e < n) w |= (uint32_t)(hash3(seed, stream, e) & 15u) << (4 * i);
  }
  out[wi] = w;
}
// I4_TGO zeros: 7 + (hash & 1) as f16.
__global__ void synth_zero_kernel(uint64_t seed, uint64_t stream, size_t n, uint16_t* out) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = f16_loader_bits((float)(7 + (hash3(seed, stream, i) & 1u)));
}
// I8 codes: hash % 255 - 127.
__global__ void synth_i8_kernel(uint64_t seed, uint64_t stream, size_t n, int8_t* out) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = (int8_t)((int)(hash3(seed, stream, i) % 255u) - 127);
}
// Norm gains: multiples of 1/8 in [-2, 2), ((hash % 32) - 16) / 8.
__global__ void synth_gain_kernel(uint64_t seed, uint64_t stream, size_t n, float* out) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = (float)((int)(hash3(seed, stream, i) % 32u) - 16) / 8.0f;
}
__global__ void fill_f32_kernel(float* p, size_t n, float v) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}
__global__ void zero_u32_kernel(uint32_t* p, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// ---- host launchers --------------------------------------------------------
static inline dim3 grid1(size_t n, int b = 256) { return dim3((unsigned)((n + b - 1) / b)); }

void launch_embed(const uint32_t* ids, int T, const void* table, const uint16_t* scales, int form,
                  int d, float* h, hipStream_t st, const int32_t* feed) {
  hipLaunchKernelGGL(embed_kernel, dim3(T), dim3(256), 0, st, ids, table, scales, form, d, h, feed);
}
void launch_rmsnorm(float* x, const uint32_t* rows, int nrows, const float* g, int w,
                    float eps, void* out, int out_form, hipStream_t st, const float* part,
                    int nsplit, size_t plane) {
  const int threads = std::min(1024, std::max(64, (w / 4 + 63) / 64 * 64));
  const int per = (w + 4 * threads - 1) / (4 * threads);  // float4s per thread
#define RMSNORM_LAUNCH(R)                                                                      \
  hipLaunchKernelGGL(rmsnorm_kernel<R>, dim3(nrows), dim3(threads), 0, st, x, rows, g, w, eps, \
                     out, out_form, part, nsplit, plane)
  if (per <= 1) RMSNORM_LAUNCH(1);
  else if (per == 2) RMSNORM_LAUNCH(2);
  else if (per <= 4) RMSNORM_LAUNCH(4);
  else RMSNORM_LAUNCH(0);
#undef RMSNORM_LAUNCH
}
__global__ __launch_bounds__(256) void rope_table_kernel(const uint32_t* rowpos, int T,
                                                        const double* inv_freq, float4_t* table) {
  const int i = blockIdx.x * 256 + threadIdx.x;  // row i / 32, frequency pair i % 32
  if (i >= T * 32) return;
  const int l = i & 31;
  const int pos = (int)rowpos[i >> 5];
  const double ang0 = (double)pos * inv_freq[2 * l], ang1 = (double)pos * inv_freq[2 * l + 1];
  table[i] = float4_t{(float)cos(ang0), (float)sin(ang0), (float)cos(ang1), (float)sin(ang1)};
}
void launch_rope_table(const uint32_t* rowpos, int T, const double* inv_freq, float4_t* table,
                       hipStream_t st) {
  if (T <= 0) return;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((T * 32 + 255) / 256)), dim3(256), 0, st,
                     rowpos, T, inv_freq, table);
}
void launch_derive_rows(const DeriveArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(derive_rows_kernel, dim3(a.B + 1), dim3(256), 0, st, a);
}
void launch_qk_rope_kv(const QKRopeArgs& a, int T, hipStream_t st) {
  // A block's 4 waves take 8 heads; enough blocks per row to fill the chip
  // when the rows are few (a decode step), one per row otherwise.
  const int groups = (a.H + 2 * a.Hkv + 7) / 8;
  const int gy = T >= 512 ? 1 : groups;
  hipLaunchKernelGGL(qk_rope_kv_kernel, dim3(T, gy), dim3(256), 0, st, a);
}
void launch_argmax(float* logits, int B, int V, const uint32_t* extents, int32_t* out,
                   void* scratch, hipStream_t st, int keep_idle, double* margin, int zero_idle,
                   int rows, const int32_t* cidx) {
  if (B <= 0) return;
  if (!cidx) rows = B;
  if (rows > 0) {
    const int S = argmax_chunks(rows, V);
    hipLaunchKernelGGL(argmax_part_kernel, dim3(rows, S), dim3(kArgmaxThreads), 0, st, logits, V,
                       S, cidx ? nullptr : extents, cidx ? 0 : zero_idle, (Top2*)scratch);
    hipLaunchKernelGGL(argmax_final_kernel, dim3((B + 63) / 64), dim3(64), 0, st, logits, B, V, S,
                       extents, (const Top2*)scratch, out, keep_idle, margin, cidx);
  } else {
    hipLaunchKernelGGL(argmax_final_kernel, dim3((B + 63) / 64), dim3(64), 0, st, logits, B, V, 1,
                       extents, (const Top2*)scratch, out, keep_idle, margin, cidx);
  }
}
void launch_synth_f16(uint64_t seed, uint64_t stream, size_t n, double sigma, uint16_t* out,
                      hipStream_t st) {
  hipLaunchKernelGGL(synth_f16_kernel, grid1(n), dim3(256), 0, st, seed, stream, n, sigma, out);
}
void launch_synth_absf16(uint64_t seed, uint64_t stream, size_t n, double sigma, uint16_t* out,
                         hipStream_t st) {
  hipLaunchKernelGGL(synth_absf16_kernel, grid1(n), dim3(256), 0, st, seed, stream, n, sigma, out);
}
void launch_synth_i4sym(uint64_t seed, uint64_t stream, int K, int N, uint32_t* out, hipStream_t st) {
  hipLaunchKernelGGL(synth_i4sym_kernel, grid1((size_t)(K / 8) * N), dim3(256), 0, st, seed, stream, K, N, out);
}
void launch_synth_i4tgo(uint64_t seed, uint64_t stream, size_t n, uint32_t* out, hipStream_t st) {
  hipLaunchKernelGGL(synth_i4tgo_kernel, grid1((n + 7) / 8), dim3(256), 0, st, seed, stream, n, out);
}
void launch_synth_zero(uint64_t seed, uint64_t stream, size_t n, uint16_t* out, hipStream_t st) {
  hipLaunchKernelGGL(synth_zero_kernel, grid1(n), dim3(256), 0, st, seed, stream, n, out);
}
void launch_synth_i8(uint64_t seed, uint64_t stream, size_t n, int8_t* out, hipStream_t st) {
  hipLaunchKernelGGL(synth_i8_kernel, grid1(n), dim3(256), 0, st, seed, stream, n, out);
}
void launch_synth_gain(uint64_t seed, uint64_t stream, size_t n, float* out, hipStream_t st) {
  hipLaunchKernelGGL(synth_gain_kernel, grid1(n), dim3(256), 0, st, seed, stream, n, out);
}
void launch_fill_f32(float* p, size_t n, float v, hipStream_t st) {
  hipLaunchKernelGGL(fill_f32_kernel, grid1(n), dim3(256), 0, st, p, n, v);
}
void launch_zero_u32(uint32_t* p, size_t n, hipStream_t st) {
  hipLaunchKernelGGL(zero_u32_kernel, grid1(n), dim3(256), 0, st, p, n);
}

}  // namespace tgohip
