// attention.hip -- ragged paged attention over an f16 KV pool, one launch for
// decode rows and prefill chunks (tensor.Attention with QueryExtents, Lengths,
// Pages, Block: nn/attention.go:234-253; semantics of
// internal/conformance/ragged_test.go:151-208).
//
// Design (CDNA4, wave64):
//  * Work items are (sequence, kv head, token range, position range), built on
//    the host from lengths/extents. A sequence's decomposition depends only on
//    its own (length, extent), so a mixed step computes bit-for-bit what the
//    same sequences compute in separate steps.
//  * A workgroup of 4 waves stages 64 positions of K and V (16 KiB each) in LDS
//    per iteration with 16-byte coalesced loads through the page table, XOR-
//    swizzled by position so MFMA operand reads are bank-conflict free. The next
//    tile's loads are in flight while the current tile is computed.
//  * Scores are S^T = K . Q^T on v_mfma_f32_16x16x32_f16 with q split into an f16
//    high and low part (two MFMAs), so the f32 query is carried to ~2^-22 and
//    the product with the f16 key is accumulated in f32. The D layout of S^T is
//    exactly the B-operand layout of O^T = V^T . P^T on v_mfma_f32_16x16x16_f16,
//    so probabilities never leave registers; the online-softmax statistics of a
//    row live in the same lanes as that row's output accumulators.
//  * Items with at most 16 rows (decodes: 1 token x G query heads) let the four
//    waves take different positions and merge in LDS; long contexts are split
//    into 512-position parts merged by a second kernel. Items with more rows
//    (prefill chunks) give each wave 32 rows and share every staged tile.
#include "../common.h"

#include <algorithm>
#include <cmath>

namespace tgohip {

struct AttnArgs {
  const void* q;
  const half_t* k;
  const half_t* v;
  void* out;
  float* part_o;   // [parts][16][128]
  float* part_ml;  // [parts][32]: m[16] then l[16]
  const AttnItem* items;
  const AttnCombine* combines;
  const int32_t* cu;
  const uint32_t* lengths;
  const uint32_t* extents;
  const uint32_t* pages;
  int q_f16, out_f16;
  int max_pages, block, H, Hkv, G;
  float qscale;  // scale * log2(e)
};

__device__ __forceinline__ float wave_max16x(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}
__device__ __forceinline__ float wave_sum16x(float v) {
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

__device__ __forceinline__ void store_out8(void* out, int f16, size_t off, const float* v) {
  if (f16) {
    half8_t h;
#pragma unroll
    for (int j = 0; j < 8; j++) h[j] = (half_t)v[j];
    *(half8_t*)((half_t*)out + off) = h;
  } else {
    float4_t a = {v[0], v[1], v[2], v[3]}, b = {v[4], v[5], v[6], v[7]};
    *(float4_t*)((float*)out + off) = a;
    *(float4_t*)((float*)out + off + 4) = b;
  }
}

__global__ __launch_bounds__(256, 3) void attn_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[32768 + 512];
  half_t* Ks = (half_t*)smem;
  half_t* Vs = (half_t*)(smem + 16384);

  const AttnItem it = a.items[blockIdx.x];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int s = it.seq, kvh = it.kvh, G = a.G;
  const int L = (int)a.lengths[s], n = (int)a.extents[s], cu = a.cu[s];
  const int R = it.ntok * G;
  const bool pmode = it.mode == 1;
  // Each wave owns one block of 16 rows: in a prefill-style item the four
  // waves own rows [16w, 16w+16); in a decode-style item all four hold the
  // same rows and take different positions.
  const int r = (pmode ? wave * 16 : 0) + li;
  const bool valid = r < R;
  const int tok = it.tok0 + (valid ? r / G : 0);
  const int head = kvh * G + (valid ? r % G : 0);
  const int lim = valid ? (L - n + tok) : -1;

  // Q as the B operand of S^T = K.Q^T: lane holds row li, dims 32c + 8lg +
  // [0,8), scaled by scale*log2(e) and split hi + lo.
  half8_t qh[4], ql[4];
  {
    const size_t qoff = ((size_t)(cu + tok) * a.H + head) * kHeadDim;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      float x[8];
      const int d0 = 32 * c + 8 * lg;
      if (valid) {
        if (a.q_f16) {
          half8_t h = *(const half8_t*)((const half_t*)a.q + qoff + d0);
#pragma unroll
          for (int j = 0; j < 8; j++) x[j] = (float)h[j];
        } else {
          float4_t u = *(const float4_t*)((const float*)a.q + qoff + d0);
          float4_t w = *(const float4_t*)((const float*)a.q + qoff + d0 + 4);
          x[0] = u[0]; x[1] = u[1]; x[2] = u[2]; x[3] = u[3];
          x[4] = w[0]; x[5] = w[1]; x[6] = w[2]; x[7] = w[3];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; j++) x[j] = 0.f;
      }
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float xs = x[j] * a.qscale;
        const half_t hi = (half_t)xs;
        qh[c][j] = hi;
        ql[c][j] = (half_t)(xs - (float)hi);
      }
    }
  }

  float m = -INFINITY, l = 0.f;
  float4_t o[8];
#pragma unroll
  for (int db = 0; db < 8; db++) o[db] = float4_t{0.f, 0.f, 0.f, 0.f};

  const uint32_t* prow = a.pages + (size_t)s * a.max_pages;
  uint4 kreg[4], vreg[4];
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = tid + 256 * i, pos = c >> 4, dch = c & 15, p = t0 + pos;
      if (p < it.kv_hi) {
        const size_t row = (size_t)prow[p / a.block] * a.block + (p % a.block);
        const size_t off = (row * a.Hkv + kvh) * kHeadDim + dch * 8;
        kreg[i] = *(const uint4*)(a.k + off);
        vreg[i] = *(const uint4*)(a.v + off);
      } else {
        kreg[i] = make_uint4(0, 0, 0, 0);
        vreg[i] = make_uint4(0, 0, 0, 0);
      }
    }
  };

  int t0 = it.kv_lo;
  if (t0 < it.kv_hi) load_tile(t0);
  for (; t0 < it.kv_hi; t0 += kAttnTile) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = tid + 256 * i, pos = c >> 4, dch = c & 15;
      const int phys = pos * 16 + (dch ^ (pos & 15));
      ((uint4*)Ks)[phys] = kreg[i];
      ((uint4*)Vs)[phys] = vreg[i];
    }
    __syncthreads();
    if (t0 + kAttnTile < it.kv_hi) load_tile(t0 + kAttnTile);

    const int mb0 = pmode ? 0 : wave, mb1 = pmode ? 4 : wave + 1;
    for (int mb = mb0; mb < mb1; mb++) {
      if (t0 + mb * 16 >= it.kv_hi) break;
      float4_t st = {0.f, 0.f, 0.f, 0.f};
      {
        const int pos = mb * 16 + li;
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const half8_t ka = *(const half8_t*)(Ks + (pos * 16 + ((4 * c + lg) ^ (pos & 15))) * 8);
          st = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[c], st, 0, 0, 0);
          st = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[c], st, 0, 0, 0);
        }
      }
      float sv[4];
      float tmax = -INFINITY;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int pabs = t0 + mb * 16 + 4 * lg + q;
        const bool ok = pabs <= lim && pabs < it.kv_hi;
        sv[q] = ok ? st[q] : -INFINITY;
        tmax = fmaxf(tmax, sv[q]);
      }
      tmax = wave_max16x(tmax);
      const float mnew = fmaxf(m, tmax);
      float alpha = 1.f;
      half4_t pb;
      float psum = 0.f;
      if (mnew == -INFINITY) {
#pragma unroll
        for (int q = 0; q < 4; q++) pb[q] = (half_t)0.f;
      } else {
        alpha = exp2f(m - mnew);
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float p = exp2f(sv[q] - mnew);
          psum += p;
          pb[q] = (half_t)p;
        }
      }
      psum = wave_sum16x(psum);
      l = l * alpha + psum;
      m = mnew;
      // O^T += V^T . P^T: the A operand holds V[pos 4lg+e][dim 16db+li].
#pragma unroll
      for (int db = 0; db < 8; db++) {
        const int d = db * 16 + li;
        half4_t va;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int pos = mb * 16 + 4 * lg + e;
          va[e] = Vs[(pos * 16 + ((d >> 3) ^ (pos & 15))) * 8 + (d & 7)];
        }
        o[db] *= alpha;
        o[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pb, o[db], 0, 0, 0);
      }
    }
  }

  if (!pmode) {
    // Merge the four waves' partial softmax states for the (up to) 16 rows.
    __syncthreads();
    float* Os = (float*)smem;               // [4][16][128]
    float* Ms = (float*)(smem + 32768);     // [4][16] m, then [4][16] l
#pragma unroll
    for (int db = 0; db < 8; db++)
#pragma unroll
      for (int q = 0; q < 4; q++) Os[(wave * 16 + li) * 128 + db * 16 + 4 * lg + q] = o[db][q];
    if (lg == 0) {
      Ms[wave * 16 + li] = m;
      Ms[64 + wave * 16 + li] = l;
    }
    __syncthreads();
    const int row = tid >> 4, d0 = (tid & 15) * 8;
    float mstar = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; w++) mstar = fmaxf(mstar, Ms[w * 16 + row]);
    float lsum = 0.f, acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const float mw = Ms[w * 16 + row];
      const float wt = (mw == -INFINITY) ? 0.f : exp2f(mw - mstar);
      lsum += wt * Ms[64 + w * 16 + row];
      const float* src = Os + (w * 16 + row) * 128 + d0;
#pragma unroll
      for (int j = 0; j < 8; j++) acc[j] += wt * src[j];
    }
    if (row < R) {
      if (it.part < 0) {
        const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) acc[j] *= inv;
        const int tk = it.tok0 + row / G, hd = kvh * G + row % G;
        store_out8(a.out, a.out_f16, ((size_t)(cu + tk) * a.H + hd) * kHeadDim + d0, acc);
      } else {
        float* po = a.part_o + ((size_t)it.part * 16 + row) * 128 + d0;
#pragma unroll
        for (int j = 0; j < 8; j++) po[j] = acc[j];
        if ((tid & 15) == 0) {
          a.part_ml[(size_t)it.part * 32 + row] = mstar;
          a.part_ml[(size_t)it.part * 32 + 16 + row] = lsum;
        }
      }
    }
  } else if (valid) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const size_t base = ((size_t)(cu + tok) * a.H + head) * kHeadDim;
#pragma unroll
    for (int db = 0; db < 8; db++) {
      const size_t off = base + db * 16 + 4 * lg;
      if (a.out_f16) {
        half4_t hv;
#pragma unroll
        for (int q = 0; q < 4; q++) hv[q] = (half_t)(o[db][q] * inv);
        *(half4_t*)((half_t*)a.out + off) = hv;
      } else {
        *(float4_t*)((float*)a.out + off) = o[db] * inv;
      }
    }
  }
}

// Merges the parts of split items in part order (deterministic).
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  const AttnCombine cb = a.combines[blockIdx.x];
  const int tid = threadIdx.x, row = tid >> 4, d0 = (tid & 15) * 8, G = a.G;
  const int R = cb.ntok * G;
  if (row >= R) return;
  float mstar = -INFINITY;
  for (int p = 0; p < cb.nparts; p++) mstar = fmaxf(mstar, a.part_ml[(size_t)(cb.part0 + p) * 32 + row]);
  float lsum = 0.f, acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int p = 0; p < cb.nparts; p++) {
    const size_t part = (size_t)(cb.part0 + p);
    const float mw = a.part_ml[part * 32 + row];
    const float wt = (mw == -INFINITY) ? 0.f : exp2f(mw - mstar);
    lsum += wt * a.part_ml[part * 32 + 16 + row];
    const float* src = a.part_o + (part * 16 + row) * 128 + d0;
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] += wt * src[j];
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
  for (int j = 0; j < 8; j++) acc[j] *= inv;
  const int tok = cb.tok0 + row / G, head = cb.kvh * G + row % G;
  store_out8(a.out, a.out_f16, ((size_t)(a.cu[cb.seq] + tok) * a.H + head) * kHeadDim + d0, acc);
}

// Zeroes rows [r0, r1) of a [T, width] activation: the inert pad rows.
__global__ void zero_rows_kernel(void* out, int f16, size_t start, size_t count) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  if (f16) ((half_t*)out)[start + i] = (half_t)0.f;
  else ((float*)out)[start + i] = 0.f;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

// Builds the work decomposition. Validates what the kernel relies on: every
// position a claimed row reads has a page-table entry inside the pool.
int attn_build_plan(int T, int B, const uint32_t* lengths, const uint32_t* extents,
                    const uint32_t* pages, int max_pages, int block, int capacity, int H,
                    int Hkv, AttnPlan& plan) {
  if (H <= 0 || Hkv <= 0 || H % Hkv != 0)
    return fail(TGOHIP_EINVAL, "attention: query heads " + std::to_string(H) +
                                   " are not a multiple of kv heads " + std::to_string(Hkv));
  const int G = H / Hkv;
  if (G > kAttnRowsP)
    return fail(TGOHIP_EINVAL, "attention: a kv head shared by more than 128 query heads");
  if (block <= 0) return fail(TGOHIP_EINVAL, "attention: block is " + std::to_string(block));
  plan.items.clear();
  plan.combines.clear();
  plan.cu.assign(B, 0);
  plan.parts = 0;
  int64_t at = 0;
  const int pool_pages = capacity / block;
  for (int s = 0; s < B; s++) {
    plan.cu[s] = (int32_t)at;
    const int64_t n = extents[s], L = lengths[s];
    if (n > L)
      return fail(TGOHIP_EINVAL, "attention: sequence " + std::to_string(s) + " has extent " +
                                     std::to_string(n) + " above its length " + std::to_string(L));
    if (n > 0) {
      const int64_t need = (L + block - 1) / block;
      if (need > max_pages)
        return fail(TGOHIP_EINVAL, "attention: sequence " + std::to_string(s) + " of length " +
                                       std::to_string(L) + " needs " + std::to_string(need) +
                                       " page-table entries and the table is " +
                                       std::to_string(max_pages) + " wide");
      for (int64_t j = 0; j < need; j++)
        if ((int64_t)pages[(size_t)s * max_pages + j] >= pool_pages)
          return fail(TGOHIP_EINVAL, "attention: sequence " + std::to_string(s) + " page " +
                                         std::to_string(j) + " is block " +
                                         std::to_string(pages[(size_t)s * max_pages + j]) +
                                         " and the pool holds " + std::to_string(pool_pages));
    }
    at += n;
  }
  if (at > T)
    return fail(TGOHIP_EINVAL, "attention: the extents sum to " + std::to_string(at) +
                                   " and q has " + std::to_string(T) + " rows");
  plan.claimed = (int)at;
  for (int s = 0; s < B; s++) {
    const int n = (int)extents[s], L = (int)lengths[s];
    if (n == 0) continue;
    if (n * G <= 16) {
      const int splits = (L + kAttnSplit - 1) / kAttnSplit;
      for (int kvh = 0; kvh < Hkv; kvh++) {
        if (splits <= 1) {
          plan.items.push_back(AttnItem{s, kvh, 0, n, 0, L, -1, 0});
        } else {
          const int part0 = plan.parts;
          for (int p = 0; p < splits; p++) {
            const int lo = p * kAttnSplit, hi = std::min(L, lo + kAttnSplit);
            plan.items.push_back(AttnItem{s, kvh, 0, n, lo, hi, plan.parts++, 0});
          }
          plan.combines.push_back(AttnCombine{s, kvh, 0, n, part0, splits, 0, 0});
        }
      }
    } else {
      const int tpi = std::max(1, kAttnRowsP / G);
      for (int t0 = 0; t0 < n; t0 += tpi) {
        const int nt = std::min(tpi, n - t0);
        const int hi = L - n + t0 + nt;
        for (int kvh = 0; kvh < Hkv; kvh++)
          plan.items.push_back(AttnItem{s, kvh, t0, nt, 0, hi, -1, 1});
      }
    }
  }
  // Heavy items first so the tail of the launch is short ones.
  std::stable_sort(plan.items.begin(), plan.items.end(), [](const AttnItem& x, const AttnItem& y) {
    const int64_t cx = (int64_t)(x.kv_hi - x.kv_lo) * (x.mode ? 8 : 1);
    const int64_t cy = (int64_t)(y.kv_hi - y.kv_lo) * (y.mode ? 8 : 1);
    return cx > cy;
  });
  return 0;
}

int attn_enqueue(const AttnPlan& plan, const AttnDevPlan& dp, const void* q, int q_f16,
                 const void* k, const void* v, void* out, int out_f16, int T, int H, int Hkv,
                 int max_pages, int block, float scale, hipStream_t stream) {
  AttnArgs a;
  a.q = q;
  a.k = (const half_t*)k;
  a.v = (const half_t*)v;
  a.out = out;
  a.part_o = dp.part_o;
  a.part_ml = dp.part_ml;
  a.items = dp.items;
  a.combines = dp.combines;
  a.cu = dp.cu;
  a.lengths = dp.lengths;
  a.extents = dp.extents;
  a.pages = dp.pages;
  a.q_f16 = q_f16;
  a.out_f16 = out_f16;
  a.max_pages = max_pages;
  a.block = block;
  a.H = H;
  a.Hkv = Hkv;
  a.G = H / Hkv;
  a.qscale = scale * 1.4426950408889634f;
  if (!plan.items.empty())
    hipLaunchKernelGGL(attn_kernel, dim3((unsigned)plan.items.size()), dim3(256), 0, stream, a);
  if (!plan.combines.empty())
    hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)plan.combines.size()), dim3(256), 0,
                       stream, a);
  if (plan.claimed < T) {
    const size_t start = (size_t)plan.claimed * H * kHeadDim;
    const size_t count = (size_t)(T - plan.claimed) * H * kHeadDim;
    hipLaunchKernelGGL(zero_rows_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0,
                       stream, out, out_f16, start, count);
  }
  TGOHIP_HIP(hipGetLastError());
  return 0;
}

}  // namespace tgohip
