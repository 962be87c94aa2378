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
//    waves take different positions and merge in LDS. Items with more rows
//    (prefill chunks) take 64 rows, 16 per wave, and share every staged tile.
//    Contexts longer than kAttnSplit positions are split into parts whose
//    partial (o, m, l) a second kernel merges in part order (deterministic).
#include "../common.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>

namespace tgohip {

struct AttnArgs {
  const void* q;
  const half_t* k;
  const half_t* v;
  void* out;
  float* part_o;   // [parts][64][128]
  float* part_ml;  // [parts][128]: m[64] then l[64]
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

constexpr int kVtStride = kAttnTile + 4;  // halves per transposed-V row (bank spread)
constexpr int kMaxItemPages = 1024;        // page indices an item stages in LDS

// BLK is the page size when it is 16 (the fast path: a 64-position tile is
// four whole pages), or 0 for any other page size.
template <int BLK>
__global__ __launch_bounds__(256, 3) void attn_kernel(AttnArgs a) {
  // Ks: 64 positions x 128 dims, 16-byte chunks XOR-swizzled by position.
  // Vt: V transposed, 128 dims x 64 positions (+4 pad): the PV A operand is
  // then one 8-byte read. pg: the item's page indices.
  __shared__ __attribute__((aligned(16))) char smem[16384 + 128 * kVtStride * 2 + kMaxItemPages * 4];
  half_t* Ks = (half_t*)smem;
  half_t* Vt = (half_t*)(smem + 16384);
  uint32_t* pg = (uint32_t*)(smem + 16384 + 128 * kVtStride * 2);

  const AttnItem it = a.items[blockIdx.x];
  if (it.mode == 2) return;  // an empty slot of the XCD-aware order
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int s = it.seq, kvh = it.kvh, G = a.G;
  const int L = (int)a.lengths[s], n = (int)a.extents[s], cu = a.cu[s];
  const int R = it.ntok * G;
  const bool pmode = it.mode == 1;
  const int r = (pmode ? wave * 16 : 0) + li;
  const bool valid = r < R;
  const int tok = it.tok0 + (valid ? r / G : 0);
  const int head = kvh * G + (valid ? r % G : 0);
  const int lim = valid ? (L - n + tok) : -1;
  const int blk = BLK ? BLK : a.block;
  const bool pow2 = (blk & (blk - 1)) == 0;
  const int bshift = pow2 ? __ffs(blk) - 1 : 0;
  // Element offsets of one layer's pool fit 32 bits (the host checks).
  const uint32_t rstride = (uint32_t)a.Hkv * kHeadDim;

  // The item's page indices, staged once (a decode part spans <= 33 pages).
  const uint32_t* prow = a.pages + (size_t)s * a.max_pages;
  const int pg0 = it.kv_lo / blk;
  const int npg = it.kv_hi > it.kv_lo ? (it.kv_hi - 1) / blk - pg0 + 1 : 0;
  const bool staged = npg <= kMaxItemPages;
  if (staged)
    for (int i = tid; i < npg; i += 256) pg[i] = prow[pg0 + i];

  // Q as the B operand of S^T = K.Q^T, scaled by scale*log2(e), hi + lo.
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
  __syncthreads();  // pg visible

  float m = -INFINITY, l = 0.f;
  float4_t o[8];
#pragma unroll
  for (int db = 0; db < 8; db++) o[db] = float4_t{0.f, 0.f, 0.f, 0.f};

  auto row_of = [&](int p) -> uint32_t {
    const int pi = pow2 ? (p >> bshift) : (p / blk);
    const int po = pow2 ? (p & (blk - 1)) : (p - pi * blk);
    const uint32_t page = staged ? pg[pi - pg0] : prow[pi];
    return page * (uint32_t)blk + (uint32_t)po;
  };
  // Per tile a thread moves K chunks of positions tid/16 + 16i and V chunks of
  // the four consecutive positions 4*(tid/16) + i, dims 8*(tid%16) + [0,8).
  const int dch = tid & 15, pgrp = tid >> 4;
  const uint32_t lane_off = (uint32_t)kvh * kHeadDim + dch * 8;
  uint4 kreg[4], vreg[4];
  auto load_tile = [&](int t0) {
    if (BLK == 16 && staged && t0 + kAttnTile <= it.kv_hi && (t0 & 15) == 0) {
      // four whole pages: page i holds K positions t0+16i+pgrp; V's four
      // consecutive positions all sit in page pgrp/4
      const int pb = (t0 >> 4) - pg0;
      const uint32_t vrow = pg[pb + (pgrp >> 2)] * 16u + (uint32_t)(4 * (pgrp & 3));
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t krow = pg[pb + i] * 16u + (uint32_t)pgrp;
        kreg[i] = *(const uint4*)(a.k + krow * rstride + lane_off);
        vreg[i] = *(const uint4*)(a.v + (vrow + i) * rstride + lane_off);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int pk = t0 + pgrp + 16 * i, pv = t0 + 4 * pgrp + i;
      if (pk < it.kv_hi) kreg[i] = *(const uint4*)(a.k + row_of(pk) * rstride + lane_off);
      else kreg[i] = make_uint4(0, 0, 0, 0);
      if (pv < it.kv_hi) vreg[i] = *(const uint4*)(a.v + row_of(pv) * rstride + lane_off);
      else vreg[i] = make_uint4(0, 0, 0, 0);
    }
  };
  // Positions every row of this item may see: the first token's limit.
  const int full_hi = min(it.kv_hi, L - n + it.tok0 + 1);

  int t0 = it.kv_lo;
  if (t0 < it.kv_hi) load_tile(t0);
  for (; t0 < it.kv_hi; t0 += kAttnTile) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int pos = pgrp + 16 * i;
      ((uint4*)Ks)[pos * 16 + (dch ^ (pos & 15))] = kreg[i];
    }
    {
      union U { uint4 u; half8_t h; };
      U v0, v1, v2, v3;
      v0.u = vreg[0]; v1.u = vreg[1]; v2.u = vreg[2]; v3.u = vreg[3];
#pragma unroll
      for (int d = 0; d < 8; d++) {
        const half4_t col = {v0.h[d], v1.h[d], v2.h[d], v3.h[d]};
        *(half4_t*)(Vt + (dch * 8 + d) * kVtStride + 4 * pgrp) = col;
      }
    }
    __syncthreads();
    if (t0 + kAttnTile < it.kv_hi) load_tile(t0 + kAttnTile);

    // Scores for this wave's 16-position blocks of the tile: decode-style items
    // take block `wave`, prefill-style items all four.
    const int mb0 = pmode ? 0 : wave, nmb = pmode ? 4 : 1;
    float4_t st[4];
    float tmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      st[j] = float4_t{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      if (j >= nmb) continue;
      const int mb = mb0 + j;
      if (t0 + mb * 16 >= it.kv_hi) continue;
      float4_t acc = {0.f, 0.f, 0.f, 0.f};
      const int pos = mb * 16 + li;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const half8_t ka = *(const half8_t*)(Ks + (pos * 16 + ((4 * c + lg) ^ (pos & 15))) * 8);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[c], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[c], acc, 0, 0, 0);
      }
      if (t0 + mb * 16 + 16 <= full_hi && valid) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
          st[j][q] = acc[q];
          tmax = fmaxf(tmax, acc[q]);
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int pabs = t0 + mb * 16 + 4 * lg + q;
          st[j][q] = (pabs <= lim && pabs < it.kv_hi) ? acc[q] : -INFINITY;
          tmax = fmaxf(tmax, st[j][q]);
        }
      }
    }
    tmax = wave_max16x(tmax);
    // Branch-free update: a row that has seen no visible position keeps
    // m = -inf, alpha = 1 and p = 0. The MFMAs below must run on every lane
    // (a lane's A operand is a head dimension, not this lane's row).
    const float mnew = fmaxf(m, tmax);
    const bool none = mnew == -INFINITY;
    const float alpha = none ? 1.f : __builtin_amdgcn_exp2f(m - mnew);
    float psum = 0.f;
    half4_t pb[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float p = none ? 0.f : __builtin_amdgcn_exp2f(st[j][q] - mnew);
        psum += p;
        pb[j][q] = (half_t)p;
      }
    psum = wave_sum16x(psum);
    l = l * alpha + psum;
    m = mnew;
#pragma unroll
    for (int db = 0; db < 8; db++) o[db] *= alpha;
    // O^T += V^T . P^T; the A operand is V^T[dim 16db+li][pos 16mb+4lg..+3].
#pragma unroll
    for (int j = 0; j < 4; j++) {
      if (j >= nmb) break;
      const int mb = mb0 + j;
      if (t0 + mb * 16 >= it.kv_hi) break;
#pragma unroll
      for (int db = 0; db < 8; db++) {
        const half4_t va = *(const half4_t*)(Vt + (db * 16 + li) * kVtStride + mb * 16 + 4 * lg);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pb[j], o[db], 0, 0, 0);
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
        float* po = a.part_o + ((size_t)it.part * 64 + row) * 128 + d0;
#pragma unroll
        for (int j = 0; j < 8; j++) po[j] = acc[j];
        if ((tid & 15) == 0) {
          a.part_ml[(size_t)it.part * 128 + row] = mstar;
          a.part_ml[(size_t)it.part * 128 + 64 + row] = lsum;
        }
      }
    }
  } else if (valid && it.part >= 0) {
    // a part of a context-split prefill item: unnormalized O and (m, l)
    float* po = a.part_o + ((size_t)it.part * 64 + r) * 128;
#pragma unroll
    for (int db = 0; db < 8; db++) *(float4_t*)(po + db * 16 + 4 * lg) = o[db];
    if (lg == 0) {
      a.part_ml[(size_t)it.part * 128 + r] = m;
      a.part_ml[(size_t)it.part * 128 + 64 + r] = l;
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

// Merges the parts of split items in part order (deterministic). One block
// per item; a thread owns 8 dims of a row, 16 rows per pass.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  const AttnCombine cb = a.combines[blockIdx.x];
  const int tid = threadIdx.x, d0 = (tid & 15) * 8, G = a.G;
  const int R = cb.ntok * G;
  for (int row = tid >> 4; row < R; row += 16) {
    float mstar = -INFINITY;
    for (int p = 0; p < cb.nparts; p++)
      mstar = fmaxf(mstar, a.part_ml[(size_t)(cb.part0 + p) * 128 + row]);
    float lsum = 0.f, acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int p = 0; p < cb.nparts; p++) {
      const size_t part = (size_t)(cb.part0 + p);
      const float mw = a.part_ml[part * 128 + row];
      const float wt = (mw == -INFINITY) ? 0.f : exp2f(mw - mstar);
      lsum += wt * a.part_ml[part * 128 + 64 + row];
      const float* src = a.part_o + (part * 64 + row) * 128 + d0;
#pragma unroll
      for (int j = 0; j < 8; j++) acc[j] += wt * src[j];
    }
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] *= inv;
    const int tok = cb.tok0 + row / G, head = cb.kvh * G + row % G;
    store_out8(a.out, a.out_f16, ((size_t)(a.cu[cb.seq] + tok) * a.H + head) * kHeadDim + d0, acc);
  }
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
    return fail(TGOHIP_EINVAL, "attention: " + std::to_string(G) + " query heads share a kv head; "
                               "at most " + std::to_string(kAttnRowsP) + " are supported");
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
  // Positions per part of a decode-style item (a multiple of the 64-position
  // tile); TGOHIP_ATTN_SPLIT overrides it for tuning.
  static const int split = [] {
    const char* e = getenv("TGOHIP_ATTN_SPLIT");
    const int v = e ? atoi(e) : kAttnSplit;
    return v >= kAttnTile ? v / kAttnTile * kAttnTile : kAttnSplit;
  }();
  for (int s = 0; s < B; s++) {
    const int n = (int)extents[s], L = (int)lengths[s];
    if (n == 0) continue;
    if (n * G <= 16) {
      // The kv heads of one part are adjacent in launch order: they read the
      // same 2 KiB position rows of the pool at about the same time.
      const int splits = (L + split - 1) / split;
      if (splits <= 1) {
        for (int kvh = 0; kvh < Hkv; kvh++) plan.items.push_back(AttnItem{s, kvh, 0, n, 0, L, -1, 0});
      } else {
        const int base = plan.parts;
        for (int p = 0; p < splits; p++) {
          const int lo = p * split, hi = std::min(L, lo + split);
          for (int kvh = 0; kvh < Hkv; kvh++)
            plan.items.push_back(AttnItem{s, kvh, 0, n, lo, hi, base + kvh * splits + p, 0});
        }
        for (int kvh = 0; kvh < Hkv; kvh++)
          plan.combines.push_back(AttnCombine{s, kvh, 0, n, base + kvh * splits, splits, 0, 0});
        plan.parts += Hkv * splits;
      }
    } else {
      // Prefill-style: 64 rows per item, and the context split into parts too,
      // so a long context is walked by many workgroups in parallel.
      const int tpi = std::max(1, kAttnRowsP / G);
      for (int t0 = 0; t0 < n; t0 += tpi) {
        const int nt = std::min(tpi, n - t0);
        const int hi = L - n + t0 + nt;
        const int splits = (hi + split - 1) / split;
        for (int kvh = 0; kvh < Hkv; kvh++) {
          if (splits <= 1) {
            plan.items.push_back(AttnItem{s, kvh, t0, nt, 0, hi, -1, 1});
          } else {
            const int part0 = plan.parts;
            for (int p = 0; p < splits; p++) {
              const int lo = p * split, h2 = std::min(hi, lo + split);
              plan.items.push_back(AttnItem{s, kvh, t0, nt, lo, h2, plan.parts++, 1});
            }
            plan.combines.push_back(AttnCombine{s, kvh, t0, nt, part0, splits, 0, 0});
          }
        }
      }
    }
  }
  // Heavy items first so the tail of the launch is short ones.
  std::stable_sort(plan.items.begin(), plan.items.end(), [](const AttnItem& x, const AttnItem& y) {
    const int64_t cx = (int64_t)(x.kv_hi - x.kv_lo) * (x.mode ? 8 : 1);
    const int64_t cy = (int64_t)(y.kv_hi - y.kv_lo) * (y.mode ? 8 : 1);
    return cx > cy;
  });
  // XCD-aware order: workgroup i is dispatched to XCD i % 8, and every
  // prefill-style item of one (sequence, kv head) re-reads the same K/V
  // stream. Route each such stream to one XCD so its L2 serves the re-reads:
  // the prefill items are dealt into 8 per-XCD queues by stream, then
  // interleaved back so that position i belongs to queue i % 8.
  {
    constexpr int kXcd = 8;
    std::vector<AttnItem> pre, rest;
    for (const AttnItem& x : plan.items) (x.mode ? pre : rest).push_back(x);
    if (!pre.empty()) {
      std::vector<std::vector<AttnItem>> q(kXcd);
      for (const AttnItem& x : pre) q[(x.seq * 131 + x.kvh) % kXcd].push_back(x);
      std::vector<AttnItem> out;
      out.reserve(plan.items.size());
      size_t taken = 0;
      std::vector<size_t> at(kXcd, 0);
      while (taken < pre.size()) {
        for (int x = 0; x < kXcd; x++) {
          if (at[x] < q[x].size()) {
            out.push_back(q[x][at[x]++]);
            taken++;
          } else if (taken < pre.size()) {
            // pad this XCD's turn with a decode item so the others keep their lanes
            if (!rest.empty()) {
              out.push_back(rest.back());
              rest.pop_back();
            } else {
              out.push_back(AttnItem{0, 0, 0, 0, 0, 0, -1, 2});  // empty item
            }
          }
        }
      }
      // trailing empty fillers are not needed
      while (!out.empty() && out.back().mode == 2) out.pop_back();
      std::reverse(rest.begin(), rest.end());
      std::stable_sort(rest.begin(), rest.end(), [](const AttnItem& x, const AttnItem& y) {
        return (x.kv_hi - x.kv_lo) > (y.kv_hi - y.kv_lo);
      });
      out.insert(out.end(), rest.begin(), rest.end());
      plan.items.swap(out);
    }
  }
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
  if (!plan.items.empty()) {
    if (block == 16)
      hipLaunchKernelGGL(attn_kernel<16>, dim3((unsigned)plan.items.size()), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL(attn_kernel<0>, dim3((unsigned)plan.items.size()), dim3(256), 0, stream, a);
  }
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
