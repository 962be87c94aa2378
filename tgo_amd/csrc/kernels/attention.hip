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
//    per iteration with 16-byte coalesced loads through the page table. K rows
//    are 256-byte bank rows with 16-byte chunks XOR-swizzled by position; V is
//    transposed on the way in, its 4-position groups XOR-swizzled by dim row.
//    Barriers order LDS only, so the next tiles' loads stay in flight.
//  * An f32 q is split into an f16 high and low part (two MFMAs), so the f32
//    query is carried to ~2^-22 and the product with the f16 key is
//    accumulated in f32. An f16 q takes one MFMA, and the scores are scaled in
//    f32 afterwards.
//  * Decode-style items (<= 16 rows: 1 token x G query heads) run S^T = K.Q^T
//    on v_mfma_f32_16x16x32_f16 and O^T = V^T.P^T on v_mfma_f32_16x16x16_f16
//    (the D layout of the first is the B layout of the second). The four waves
//    take different positions, merge in LDS, and keep kDecodeDepth tiles of
//    loads in flight.
//  * Prefill-style items take 128 rows (32 tokens x 4 heads), 32 per wave, on
//    v_mfma_f32_32x32x16_f16 for both products; probabilities stay in
//    registers (see attn_prefill).
//  * Contexts longer than kAttnSplitDecode / kAttnSplitPrefill positions are
//    split into parts whose partial (o, m, l) a second kernel merges in part
//    order (deterministic). An in-kernel merge by the last part to arrive was
//    measured slower: making a partial visible across XCDs takes a
//    device-scope fence, which writes back the XCD's L2.
//  * Launch order interleaves the two kinds of item (HBM-bound decode streams
//    beside MFMA-bound prefill tiles) and routes each prefill stream to one
//    XCD so its L2 serves the re-reads.
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
  const int32_t* seqlist;
  const int32_t* cu;
  const uint32_t* lengths;
  const uint32_t* extents;
  const uint32_t* pages;
  int q_f16, out_f16;  // out_f16: OUT_F32, OUT_F16 or OUT_X2
  size_t out_lo;       // OUT_X2: elements from the hi plane to the lo plane (T * H * 128)
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

// Eight output values as f32, f16, or (OUT_X2) the f16 hi plane plus the lo
// plane f16(v - hi) lo elements further on: the activation pair the exact
// projections read.
__device__ __forceinline__ void store_out8(void* out, int f16, size_t off, const float* v,
                                           size_t lo = 0) {
  if (f16) {
    half8_t h;
#pragma unroll
    for (int j = 0; j < 8; j++) h[j] = (half_t)v[j];
    *(half8_t*)((half_t*)out + off) = h;
    if (f16 == OUT_X2) {
      half8_t l;
#pragma unroll
      for (int j = 0; j < 8; j++) l[j] = (half_t)(v[j] - (float)h[j]);
      *(half8_t*)((half_t*)out + lo + off) = l;
    }
  } else {
    float4_t a = {v[0], v[1], v[2], v[3]}, b = {v[4], v[5], v[6], v[7]};
    *(float4_t*)((float*)out + off) = a;
    *(float4_t*)((float*)out + off + 4) = b;
  }
}

// One lane's 16-byte chunk of a K or V row. A native vector (not HIP's struct
// uint4): copies through it are plain loads and stores, so the arrays of
// chunks a wave keeps in flight stay in registers.
typedef uint32_t kv16_t __attribute__((ext_vector_type(4)));
// A decode item's K/V rows are read once per launch: non-temporal loads (the
// nt bit) stream them. A plain 4 GiB read on this part runs at 6.2 TB/s with
// ordinary 16-byte loads and 7.0 TB/s with nt ones; the C4 step's attention
// launch went from 4.4-4.5 to 5.0-5.2 TB/s (decode-only step 5.1-5.3 to
// 5.9-6.0). Prefill items keep ordinary loads: the items of one (sequence,
// kv head) re-read the same K/V through their XCD's L2, and nt loads there
// cost the C4 step 2.5%.
__device__ __forceinline__ kv16_t kv_load_nt(const half_t* p) {
  return __builtin_nontemporal_load((const kv16_t*)p);
}
// A decode item over pages other sequences also read (a shared prefix
// without the cascade) keeps ordinary loads, so the caches serve the other
// sequences' reads of the same pages: with non-temporal loads the config-5
// shape without the cascade took 0.50 ms per launch instead of 0.44.
template <bool SHARED>
__device__ __forceinline__ kv16_t kv_load_dec(const half_t* p) {
  if constexpr (SHARED) return *(const kv16_t*)p;
  else return kv_load_nt(p);
}

constexpr int kMaxItemPages = 1024;        // page indices an item stages in LDS
constexpr int kAttnVBytes = 20480;         // one V tile in LDS (64 padded rows)
constexpr int kAttnSmem = 16384 + kAttnVBytes + kMaxItemPages * 4;

// V tiles live in LDS row-major, 256 bytes per position at a row pitch of
// 320 bytes, nudged by 32 bytes when bit 2 of the position is set and by 16
// when bit 3 is: the 16-byte bank slot of (position p, chunk c) is then
// (4(p&3) + 2((p>>2)&1) + ((p>>3)&1) + c) mod 16, so the 16-lane stores of one
// position and the transposing operand reads below (8 positions x 2 chunks,
// or 4 positions x 4 chunks per 32 lanes) touch distinct slots. The offset is
// additive in multiples of 16 positions and in the dim, so each lane needs one
// address register. Offset in halves of (position p, dim d):
__device__ __forceinline__ int v_off(int p, int d) {
  return 160 * p + 16 * ((p >> 2) & 1) + 8 * ((p >> 3) & 1) + d;
}

// The A operand of O^T = V^T.P^T, four positions of one dim per lane, read
// straight from row-major V with gfx950's transposing LDS read: in each
// 16-lane group, lane j names the 8 bytes at V[p0 + j/4][d0 + 4(j%4)], and
// lane i receives V[p0 + k][d0 + i] for k = 0..3.
__device__ __forceinline__ half4_t attn_vt4(const half_t* Vs, int p0, int d0, int j) {
  typedef short short4_t __attribute__((ext_vector_type(4)));
  const short4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) short4_t*)(Vs + v_off(p0 + (j >> 2), d0 + 4 * (j & 3))));
  return __builtin_bit_cast(half4_t, r);
}

// A workgroup barrier that orders LDS only: global loads in flight stay in
// flight across it (__syncthreads would wait for them).
__device__ __forceinline__ void attn_lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// What every work item shares: where its sequence, pages and tiles are.
struct AttnCtx {
  int s, kvh, G, L, n, cu;
  int blk, bshift;
  bool pow2, staged;
  int pg0;
  uint32_t rstride;          // elements per pool row (Hkv * 128)
  const uint32_t* prow;      // the sequence's page-table row
  const uint32_t* pg;        // staged page indices (LDS)
  uint32_t lane_off;         // this thread's element offset inside a pool row
  int dch, pgrp;             // this thread's 16-byte chunk and position group
};

__device__ __forceinline__ uint32_t attn_row_of(const AttnCtx& c, int p) {
  const int pi = c.pow2 ? (p >> c.bshift) : (p / c.blk);
  const int po = c.pow2 ? (p & (c.blk - 1)) : (p - pi * c.blk);
  const uint32_t page = c.staged ? c.pg[pi - c.pg0] : c.prow[pi];
  return page * (uint32_t)c.blk + (uint32_t)po;
}

// Loads one 64-position tile into registers: K chunks of positions
// pgrp + 16i, V chunks of the four consecutive positions 4*pgrp + i, dims
// 8*dch + [0,8). Positions at or past hi load zeros.
template <int BLK>
__device__ __forceinline__ void attn_load_tile(const AttnArgs& a, const AttnCtx& c, int t0, int hi,
                                               kv16_t (&kr)[4], kv16_t (&vr)[4]) {
  if (BLK == 16 && c.staged && t0 + kAttnTile <= hi && (t0 & 15) == 0) {
    // four whole pages: page i holds K positions t0+16i+pgrp; V's four
    // consecutive positions all sit in page pgrp/4
    const int pb = (t0 >> 4) - c.pg0;
    const uint32_t vrow = c.pg[pb + (c.pgrp >> 2)] * 16u + (uint32_t)(4 * (c.pgrp & 3));
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t krow = c.pg[pb + i] * 16u + (uint32_t)c.pgrp;
      kr[i] = *(const kv16_t*)(a.k + krow * c.rstride + c.lane_off);
      vr[i] = *(const kv16_t*)(a.v + (vrow + i) * c.rstride + c.lane_off);
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int pk = t0 + c.pgrp + 16 * i, pv = t0 + 4 * c.pgrp + i;
    kr[i] = pk < hi ? *(const kv16_t*)(a.k + attn_row_of(c, pk) * c.rstride + c.lane_off)
                    : kv16_t{0u, 0u, 0u, 0u};
    vr[i] = pv < hi ? *(const kv16_t*)(a.v + attn_row_of(c, pv) * c.rstride + c.lane_off)
                    : kv16_t{0u, 0u, 0u, 0u};
  }
}

// Writes a loaded tile to LDS: K row-major, one 256-byte bank row per
// position, 16-byte chunks XOR-swizzled by position; V row-major in padded
// rows (v_off).
__device__ __forceinline__ void attn_store_tile(const AttnCtx& c, half_t* Ks, half_t* Vs,
                                                const kv16_t (&kr)[4], const kv16_t (&vr)[4]) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int pos = c.pgrp + 16 * i;
    ((kv16_t*)Ks)[pos * 16 + (c.dch ^ (pos & 15))] = kr[i];
    const int pv = 4 * c.pgrp + i;
    *(kv16_t*)(Vs + v_off(pv, 8 * c.dch)) = vr[i];
  }
}

// A decode wave's own 16 positions p0 + [0,16) of a tile: lane (dch, prow) =
// (lane % 16, lane / 16) loads K positions p0 + prow + 4i and V positions
// p0 + 4prow + i, dims 8*dch + [0,8). Positions at or past hi load zeros.
template <int BLK, bool SHARED>
__device__ __forceinline__ void attn_load_block(const AttnArgs& a, const AttnCtx& c, int p0, int hi,
                                                int prow, kv16_t (&kr)[4], kv16_t (&vr)[4]) {
  if (BLK == 16) {
    // Branch-free, so the compiler can count each block's loads and wait for
    // the oldest block only (with branches here it waits for every load in
    // flight). The page table is staged in LDS (the host splits items so that
    // it always is). Positions at or past hi read position hi - 1: finite
    // values whose scores the caller masks, so their probabilities are zero.
    const int last = hi - 1;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int pk = min(p0 + prow + 4 * i, last), pv = min(p0 + 4 * prow + i, last);
      const int ik = min((pk >> 4) - c.pg0, kMaxItemPages - 1);
      const int iv = min((pv >> 4) - c.pg0, kMaxItemPages - 1);
      const uint32_t krow = c.pg[ik] * 16u + (uint32_t)(pk & 15);
      const uint32_t vrow = c.pg[iv] * 16u + (uint32_t)(pv & 15);
      kr[i] = kv_load_dec<SHARED>(a.k + krow * c.rstride + c.lane_off);
      vr[i] = kv_load_dec<SHARED>(a.v + vrow * c.rstride + c.lane_off);
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int pk = p0 + prow + 4 * i, pv = p0 + 4 * prow + i;
    kr[i] = pk < hi ? kv_load_dec<SHARED>(a.k + attn_row_of(c, pk) * c.rstride + c.lane_off)
                    : kv16_t{0u, 0u, 0u, 0u};
    vr[i] = pv < hi ? kv_load_dec<SHARED>(a.v + attn_row_of(c, pv) * c.rstride + c.lane_off)
                    : kv16_t{0u, 0u, 0u, 0u};
  }
}

// Writes a decode wave's block to its own LDS region (K rows swizzled as in
// attn_store_tile, V rows at the v_off pitch). Only this wave reads it, and a
// wave's LDS operations complete in order, so no barrier is needed.
__device__ __forceinline__ void attn_store_block(half_t* Kw, half_t* Vw, int dch, int prow,
                                                 const kv16_t (&kr)[4], const kv16_t (&vr)[4]) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int pk = prow + 4 * i;
    ((kv16_t*)Kw)[pk * 16 + (dch ^ pk)] = kr[i];
    *(kv16_t*)(Vw + v_off(4 * prow + i, 8 * dch)) = vr[i];
  }
}

// f32 q: times scale*log2(e), split into an f16 high and low part (two
// MFMAs carry about 22 bits). f16 q (QF16): the stored halves as they are, one
// MFMA; the scores are scaled in f32 instead (attn_qscale), so the product is
// the exact f32 dot product of the f16 query and key, scaled once.
template <bool QF16>
__device__ __forceinline__ void attn_load_q(const AttnArgs& a, size_t off, bool valid, half8_t& hi,
                                            half8_t& lo) {
  if (QF16) {
    if (valid) {
      hi = *(const half8_t*)((const half_t*)a.q + off);
    } else {
#pragma unroll
      for (int j = 0; j < 8; j++) hi[j] = (half_t)0.f;
    }
    lo = hi;  // unused
    return;
  }
  float x[8];
  if (valid) {
    const float4_t u = *(const float4_t*)((const float*)a.q + off);
    const float4_t w = *(const float4_t*)((const float*)a.q + off + 4);
    x[0] = u[0]; x[1] = u[1]; x[2] = u[2]; x[3] = u[3];
    x[4] = w[0]; x[5] = w[1]; x[6] = w[2]; x[7] = w[3];
  } else {
#pragma unroll
    for (int j = 0; j < 8; j++) x[j] = 0.f;
  }
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const float xs = x[j] * a.qscale;
    const half_t h = (half_t)xs;
    hi[j] = h;
    lo[j] = (half_t)(xs - (float)h);
  }
}

// What a raw score is multiplied by to reach log2 units: 1 when q carried the
// scale in (f32 q), scale*log2(e) for f16 q. Applied as exp2(fma(s, qs, -m))
// and to the tile maximum, so it costs no instruction per score.
template <bool QF16>
__device__ __forceinline__ float attn_qscale(const AttnArgs& a) {
  return QF16 ? a.qscale : 1.f;
}

// f(std::integral_constant<int, i>) for i = 0..N-1, in order: loop indices that
// are constants from the start, so arrays indexed by them stay in registers
// whatever the unroller decides.
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (N > 0) {
    static_for<N - 1>(f);
    f(std::integral_constant<int, N - 1>{});
  }
}

// Blocks of loads a decode-style item keeps in flight beside the one it
// computes on. With the non-temporal K/V loads one is enough (a CU's 8 waves
// then hold 64 KiB in flight, 16 MiB over the chip): against 3 (the depth
// with ordinary loads) the decode-only step went from 10.26-10.28 to
// 10.02-10.05 ms with 2 and to 10.00-10.05 with 1 (10.21-10.24 with 2 on
// that box), and the mixed step was the same with 1 and 2 and 1% slower
// with 3.
#ifndef TGOHIP_DECODE_DEPTH
#define TGOHIP_DECODE_DEPTH 1
#endif
constexpr int kDecodeDepth = TGOHIP_DECODE_DEPTH;

// Online softmax with a lazy reference maximum: a row's m starts at kNoMax (a
// finite "nothing seen", so masked scores of -inf give exp2 = 0 without a
// select) and moves only when a tile's maximum exceeds it by more than
// kLazyMax (log2 units). Probabilities then stay below 2^kLazyMax, well inside
// f16, and most tiles skip rescaling the accumulators; the result is the same
// softmax, normalised by a sum taken against the same m.
constexpr float kNoMax = -1.0e30f;
constexpr float kLazyMax = 8.f;

// Decode-style item (at most 16 rows: the G query heads of <= 16/G tokens).
// The four waves take the four 16-position blocks of each 64-position tile and
// merge their softmax states at the end. kDecodeDepth tiles of loads are in
// flight.
// SHARED: the item's positions include pages other sequences read too
// (ordinary loads); otherwise non-temporal ones.
template <int BLK, bool QF16, bool SHARED>
__device__ __forceinline__ void attn_decode(const AttnArgs& a, const AttnItem& it, const AttnCtx& c,
                                            char* smem) {
  const float qs = attn_qscale<QF16>(a);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  // Wave w owns positions 16w + [0,16) of every tile, in an LDS region of its
  // own: 16 K rows of 256 bytes, 16 V rows at a 320-byte pitch.
  half_t* Kw = (half_t*)smem + wave * 16 * kHeadDim;
  half_t* Vw = (half_t*)(smem + 16384) + wave * (kAttnVBytes / 8);
  const int G = c.G, R = it.ntok * G;
  const int r = li;
  const bool valid = r < R;
  const int tok = it.tok0 + (valid ? r / G : 0);
  const int head = c.kvh * G + (valid ? r % G : 0);
  const int lim = valid ? (c.L - c.n + tok) : -1;

  // Q as the B operand of S^T = K.Q^T (v_mfma_f32_16x16x32_f16): lane (li, lg)
  // holds dims 32c + 8lg + [0,8) of row li.
  half8_t qh[4], ql[4];
  {
    const size_t qoff = ((size_t)(c.cu + tok) * a.H + head) * kHeadDim;
#pragma unroll
    for (int cc = 0; cc < 4; cc++) attn_load_q<QF16>(a, qoff + 32 * cc + 8 * lg, valid, qh[cc], ql[cc]);
  }

  float m = kNoMax, l = 0.f;
  float4_t o[8];
#pragma unroll
  for (int db = 0; db < 8; db++) o[db] = float4_t{0.f, 0.f, 0.f, 0.f};
  const int full_hi = min(it.kv_hi, c.L - c.n + it.tok0 + 1);

  constexpr int D = kDecodeDepth;
  const int wofs = 16 * wave;
  kv16_t kr[D][4], vr[D][4];
  // With page 16 the block loads are issued unconditionally, the ones past the
  // item's end reading its last position again (cache hits): every step then
  // issues the same loads, the compiler can count them, and a step waits for
  // its own block only, with D - 1 blocks still in flight.
  constexpr bool kAlways = BLK == 16;
  static_for<D>([&](auto uc) {
    constexpr int u = decltype(uc)::value;
    if (kAlways || it.kv_lo + u * kAttnTile < it.kv_hi)
      attn_load_block<BLK, SHARED>(a, c, it.kv_lo + u * kAttnTile + wofs, it.kv_hi, lg, kr[u], vr[u]);
  });
  for (int tt = it.kv_lo; tt < it.kv_hi; tt += D * kAttnTile) {
    static_for<D>([&](auto uc) {
      constexpr int u = decltype(uc)::value;
      const int t0 = tt + u * kAttnTile;
      if (t0 < it.kv_hi) attn_store_block(Kw, Vw, li, lg, kr[u], vr[u]);
      if (kAlways || t0 + D * kAttnTile < it.kv_hi)
        attn_load_block<BLK, SHARED>(a, c, t0 + D * kAttnTile + wofs, it.kv_hi, lg, kr[u], vr[u]);
      if (t0 < it.kv_hi) {

        // Scores of this wave's 16-position block.
        const int mb = wave;
        float4_t st = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        if (t0 + mb * 16 < it.kv_hi) {
          float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int cc = 0; cc < 4; cc++) {
            const half8_t ka = *(const half8_t*)(Kw + (li * 16 + ((4 * cc + lg) ^ li)) * 8);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[cc], acc, 0, 0, 0);
            if (!QF16) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[cc], acc, 0, 0, 0);
          }
          if (t0 + mb * 16 + 16 <= full_hi && valid) {
            st = acc;
          } else {
#pragma unroll
            for (int q = 0; q < 4; q++) {
              const int pabs = t0 + mb * 16 + 4 * lg + q;
              st[q] = (pabs <= lim && pabs < it.kv_hi) ? acc[q] : -INFINITY;
            }
          }
        }
        float tmax = fmaxf(fmaxf(st[0], st[1]), fmaxf(st[2], st[3]));
        tmax = wave_max16x(tmax) * qs;
        // A row that has seen no visible position keeps m = kNoMax and gets
        // p = 0. The MFMAs below run on every lane.
        const bool grow = tmax > m + kLazyMax;
        if (__builtin_amdgcn_ballot_w64(grow)) {  // uniform across the wave
          const float mnew = grow ? tmax : m;
          const float alpha = __builtin_amdgcn_exp2f(m - mnew);
          l *= alpha;
#pragma unroll
          for (int db = 0; db < 8; db++) o[db] *= alpha;
          m = mnew;
        }
        float psum = 0.f;
        half4_t pb, pl;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float p = __builtin_amdgcn_exp2f(fmaf(st[q], qs, -m));
          psum += p;
          pb[q] = (half_t)p;
          // f32 q (tgo's arithmetic): P as f16 hi + lo, so V is weighted by
          // the f32 probability the normalizer l sums
          if (!QF16) pl[q] = (half_t)(p - (float)pb[q]);
        }
        psum = wave_sum16x(psum);
        l += psum;
        if (t0 + mb * 16 < it.kv_hi) {
          // O^T += V^T . P^T; the A operand is V^T[dim 16db+li][pos 16mb+4lg..+3].
#pragma unroll
          for (int db = 0; db < 8; db++) {
            const half4_t va = attn_vt4(Vw, 4 * lg, db * 16, li);
            o[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pb, o[db], 0, 0, 0);
            if (!QF16) o[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pl, o[db], 0, 0, 0);
          }
        }
      }
    });
  }

  // Merge the four waves' partial softmax states for the (up to) 16 rows.
  attn_lds_barrier();
  // Os rows are padded to 132 floats so the 16 rows a store instruction
  // touches land on distinct banks.
  constexpr int kOs = 132;
  float* Os = (float*)smem;                        // [4][16][kOs]
  float* Ms = (float*)(smem + 4 * 16 * kOs * 4);   // [4][16] m, then [4][16] l
#pragma unroll
  for (int db = 0; db < 8; db++) *(float4_t*)(Os + (wave * 16 + li) * kOs + db * 16 + 4 * lg) = o[db];
  if (lg == 0) {
    Ms[wave * 16 + li] = l > 0.f ? m : -INFINITY;
    Ms[64 + wave * 16 + li] = l;
  }
  attn_lds_barrier();
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
    const float* src = Os + (w * 16 + row) * kOs + d0;
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] += wt * src[j];
  }
  if (row < R) {
    if (it.part < 0) {
      const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
      for (int j = 0; j < 8; j++) acc[j] *= inv;
      const int tk = it.tok0 + row / G, hd = c.kvh * G + row % G;
      store_out8(a.out, a.out_f16, ((size_t)(c.cu + tk) * a.H + hd) * kHeadDim + d0, acc, a.out_lo);
    } else {
      float* po = a.part_o + ((size_t)it.part * kAttnRowsP + row) * 128 + d0;
#pragma unroll
      for (int j = 0; j < 8; j++) po[j] = acc[j];
      if ((tid & 15) == 0) {
        a.part_ml[(size_t)it.part * 2 * kAttnRowsP + row] = mstar;
        a.part_ml[(size_t)it.part * 2 * kAttnRowsP + kAttnRowsP + row] = lsum;
      }
    }
  }
}

// Prefill-style item (up to 128 rows = 32 tokens x 4 query heads): wave w owns
// rows 32w + [0,32) and every wave consumes every staged tile.
//   S^T = K . Q^T on v_mfma_f32_32x32x16_f16: A = K (32 positions x 16 dims,
//   lane (p, kh) reads position p, dims 16s + 8kh + [0,8)), B = Q^T from
//   registers (hi + lo for an f32 q, the f16 q itself with QF16). Lane (r, kh)
//   gets the scores of row r at positions
//   8(i/4) + 4kh + i%4, i = 0..15, of each 32-position block.
//   O^T += V^T . P^T on the same MFMA: its k index 8kh + e maps to position
//   16t + (e < 4 ? 4kh + e : 8 + 4kh + e - 4) of the block, which is exactly
//   where the lane's own probabilities sit (scores i = 8t..8t+7), so P never
//   leaves registers; the A operand is two 8-byte reads of transposed V.
template <int BLK, bool QF16>
__device__ __forceinline__ void attn_prefill(const AttnArgs& a, const AttnItem& it, const AttnCtx& c,
                                             char* smem) {
  const float qs = attn_qscale<QF16>(a);
  half_t* Ks = (half_t*)smem;
  half_t* Vs = (half_t*)(smem + 16384);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, kh = lane >> 5;
  const int G = c.G, R = it.ntok * G;
  const int r = wave * 32 + l32;
  const bool valid = r < R;
  // A shared-prefix item's rows are the decode tokens of several sequences,
  // each of which sees every prefix position.
  const bool shared = it.mode == 3;
  const int rseq = shared ? a.seqlist[it.tok0 + (valid ? r / G : 0)] : c.s;
  const int tok = shared ? 0 : it.tok0 + (valid ? r / G : 0);
  const int head = c.kvh * G + (valid ? r % G : 0);
  const int lim = !valid ? -1 : shared ? it.kv_hi : (c.L - c.n + tok);
  // Positions every valid row of this wave may see (its first token's limit),
  // and whether the wave's rows are all valid.
  const int wtok0 = it.tok0 + (wave * 32) / G;
  const int wave_hi = shared ? it.kv_hi : min(it.kv_hi, c.L - c.n + wtok0 + 1);
  const bool wave_full = wave * 32 + 32 <= R;
  const int rcu = shared ? a.cu[rseq] : c.cu;

  half8_t qh[8], ql[8];
  {
    const size_t qoff = ((size_t)(rcu + tok) * a.H + head) * kHeadDim;
#pragma unroll
    for (int ss = 0; ss < 8; ss++) attn_load_q<QF16>(a, qoff + 16 * ss + 8 * kh, valid, qh[ss], ql[ss]);
  }

  float m = kNoMax, l = 0.f;
  float16_t o[4];
#pragma unroll
  for (int db = 0; db < 4; db++)
#pragma unroll
    for (int i = 0; i < 16; i++) o[db][i] = 0.f;

  kv16_t kr[4], vr[4];
  if (it.kv_lo < it.kv_hi) attn_load_tile<BLK>(a, c, it.kv_lo, it.kv_hi, kr, vr);
  for (int t0 = it.kv_lo; t0 < it.kv_hi; t0 += kAttnTile) {
    attn_lds_barrier();
    attn_store_tile(c, Ks, Vs, kr, vr);
    attn_lds_barrier();
    if (t0 + kAttnTile < it.kv_hi) attn_load_tile<BLK>(a, c, t0 + kAttnTile, it.kv_hi, kr, vr);
    float16_t sc[2];
#pragma unroll
    for (int pb = 0; pb < 2; pb++) {
      float16_t acc;
#pragma unroll
      for (int i = 0; i < 16; i++) acc[i] = 0.f;
      const int pos = pb * 32 + l32;
#pragma unroll
      for (int ss = 0; ss < 8; ss++) {
        const half8_t ka = *(const half8_t*)(Ks + (pos * 16 + ((2 * ss + kh) ^ (pos & 15))) * 8);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qh[ss], acc, 0, 0, 0);
        if (!QF16) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, ql[ss], acc, 0, 0, 0);
      }
      sc[pb] = acc;
    }
    float tmax = -INFINITY;
    if (wave_full && t0 + kAttnTile <= wave_hi) {
#pragma unroll
      for (int pb = 0; pb < 2; pb++)
#pragma unroll
        for (int i = 0; i < 16; i++) tmax = fmaxf(tmax, sc[pb][i]);
    } else {
#pragma unroll
      for (int pb = 0; pb < 2; pb++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const int p = t0 + pb * 32 + 8 * (i >> 2) + 4 * kh + (i & 3);
          if (!(p <= lim && p < it.kv_hi)) sc[pb][i] = -INFINITY;
          tmax = fmaxf(tmax, sc[pb][i]);
        }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64)) * qs;
    const bool grow = tmax > m + kLazyMax;
    if (__builtin_amdgcn_ballot_w64(grow)) {  // uniform across the wave
      const float mnew = grow ? tmax : m;
      const float alpha = __builtin_amdgcn_exp2f(m - mnew);
      l *= alpha;
#pragma unroll
      for (int db = 0; db < 4; db++) o[db] *= alpha;
      m = mnew;
    }
    float psum = 0.f;
    half8_t pf[2][2], pfl[2][2];
#pragma unroll
    for (int pb = 0; pb < 2; pb++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const float p = __builtin_amdgcn_exp2f(fmaf(sc[pb][i], qs, -m));
        psum += p;
        const half_t ph = (half_t)p;
        pf[pb][i >> 3][i & 7] = ph;
        if (!QF16) pfl[pb][i >> 3][i & 7] = (half_t)(p - (float)ph);  // P as hi + lo (f32 q)
      }
    psum += __shfl_xor(psum, 32, 64);
    l += psum;
    // The PV operand of lane (l32, kh): dim 32db + l32, positions
    // 32pb + 16t + 4kh + [0,4) and the same + 8 -- two transposing reads whose
    // 16-lane groups take dims 32db + 16*(l32/16) + [0,16).
    const int j16 = lane & 15, dgrp = 16 * ((lane >> 4) & 1);
#pragma unroll
    for (int pb = 0; pb < 2; pb++)
#pragma unroll
      for (int t = 0; t < 2; t++) {
        const int p0 = pb * 32 + 16 * t + 4 * kh;
#pragma unroll
        for (int db = 0; db < 4; db++) {
          const half4_t v0 = attn_vt4(Vs, p0, db * 32 + dgrp, j16);
          const half4_t v1 = attn_vt4(Vs, p0 + 8, db * 32 + dgrp, j16);
          const half8_t va = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pf[pb][t], o[db], 0, 0, 0);
          if (!QF16) o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pfl[pb][t], o[db], 0, 0, 0);
        }
      }
  }

  if (!valid) return;
  // Lane (r, kh) holds dims 32db + 8g + 4kh + [0,4) of row r, g = 0..3.
  if (it.part < 0) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const size_t base = ((size_t)(rcu + tok) * a.H + head) * kHeadDim;
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const size_t off = base + db * 32 + 8 * g + 4 * kh;
        if (a.out_f16) {
          half4_t hv;
#pragma unroll
          for (int q = 0; q < 4; q++) hv[q] = (half_t)(o[db][4 * g + q] * inv);
          *(half4_t*)((half_t*)a.out + off) = hv;
          if (a.out_f16 == OUT_X2) {
            half4_t lv;
#pragma unroll
            for (int q = 0; q < 4; q++) lv[q] = (half_t)(o[db][4 * g + q] * inv - (float)hv[q]);
            *(half4_t*)((half_t*)a.out + a.out_lo + off) = lv;
          }
        } else {
          const float4_t fv = {o[db][4 * g] * inv, o[db][4 * g + 1] * inv, o[db][4 * g + 2] * inv,
                               o[db][4 * g + 3] * inv};
          *(float4_t*)((float*)a.out + off) = fv;
        }
      }
  } else {
    float* po = a.part_o + ((size_t)it.part * kAttnRowsP + r) * 128;
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const float4_t fv = {o[db][4 * g], o[db][4 * g + 1], o[db][4 * g + 2], o[db][4 * g + 3]};
        *(float4_t*)(po + db * 32 + 8 * g + 4 * kh) = fv;
      }
    if (kh == 0) {
      a.part_ml[(size_t)it.part * 2 * kAttnRowsP + r] = l > 0.f ? m : -INFINITY;
      a.part_ml[(size_t)it.part * 2 * kAttnRowsP + kAttnRowsP + r] = l;
    }
  }
}

// BLK is the page size when it is 16 (the fast path: a 64-position tile is
// four whole pages), or 0 for any other page size.
// DEC: a launch of decode-style items only (a decode-only step). Without the
// prefill path the kernel fits 128 VGPRs instead of 218, so four workgroups
// share a CU instead of two: the C4 decode-only step's attention launch
// 0.1634-0.1638 -> 0.1622-0.1624 ms (three alternating pairs). With an f32
// query (q and P as hi + lo) it needs 152 and three share a CU.
template <int BLK, bool QF16, bool DEC = false>
__global__ __launch_bounds__(256, DEC ? (QF16 ? 4 : 3) : 2) void attn_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[kAttnSmem];
  const AttnItem it = a.items[blockIdx.x];
  if (it.mode == 2) return;  // an empty slot of the XCD-aware order
  const int tid = threadIdx.x;
  AttnCtx c;
  c.s = it.seq;
  c.kvh = it.kvh;
  c.G = a.G;
  c.L = (int)a.lengths[c.s];
  c.n = (int)a.extents[c.s];
  c.cu = a.cu[c.s];
  c.blk = BLK ? BLK : a.block;
  c.pow2 = (c.blk & (c.blk - 1)) == 0;
  c.bshift = c.pow2 ? __ffs(c.blk) - 1 : 0;
  // Element offsets of one layer's pool fit 32 bits (the host checks).
  c.rstride = (uint32_t)a.Hkv * kHeadDim;
  c.prow = a.pages + (size_t)c.s * a.max_pages;
  uint32_t* pg = (uint32_t*)(smem + 16384 + kAttnVBytes);
  c.pg = pg;
  c.pg0 = it.kv_lo / c.blk;
  const int npg = it.kv_hi > it.kv_lo ? (it.kv_hi - 1) / c.blk - c.pg0 + 1 : 0;
  c.staged = npg <= kMaxItemPages;
  if (c.staged)
    for (int i = tid; i < npg; i += 256) pg[i] = c.prow[c.pg0 + i];
  c.dch = tid & 15;
  c.pgrp = tid >> 4;
  c.lane_off = (uint32_t)c.kvh * kHeadDim + c.dch * 8;
  __syncthreads();  // pg visible
  if constexpr (DEC) {
    if (it.mode & kAttnSharedPages) attn_decode<BLK, QF16, true>(a, it, c, smem);
    else attn_decode<BLK, QF16, false>(a, it, c, smem);
  } else if ((it.mode & kAttnModeMask) == 0) {
    // Decode waves are HBM streams: raised priority lets their loads and short
    // softmax steps issue ahead of a co-resident prefill item's MFMA work.
    __builtin_amdgcn_s_setprio(1);
    if (it.mode & kAttnSharedPages) attn_decode<BLK, QF16, true>(a, it, c, smem);
    else attn_decode<BLK, QF16, false>(a, it, c, smem);
  } else {
    attn_prefill<BLK, QF16>(a, it, c, smem);
  }
}

// Merges the parts of split items in part order (deterministic). A block
// takes 16 rows of an item; a thread owns 8 dims of a row.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  const AttnCombine cb = a.combines[blockIdx.x];
  const int tid = threadIdx.x, d0 = (tid & 15) * 8, G = a.G;
  const int R = cb.ntok * G;
  {
    const int row = (int)blockIdx.y * 16 + (tid >> 4);  // 16 rows per block
    if (row >= R) return;
    // parts in merge order: the shared prefix's (at row xrow + row), then the
    // sequence's own (at row)
    const int np = cb.xparts + cb.nparts;
    // One pass in part order: a part's (m, l, o) are read together (no load
    // waits for an earlier part's) and folded into a running state kept at
    // the running maximum, as an online softmax folds tiles.
    float m = -INFINITY, lsum = 0.f, acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int p = 0; p < np; p++) {
      const size_t part = (size_t)(p < cb.xparts ? cb.xpart0 + p : cb.part0 + p - cb.xparts);
      const int pr = p < cb.xparts ? cb.xrow + row : row;
      const float mp = a.part_ml[part * 2 * kAttnRowsP + pr];
      const float lp = a.part_ml[part * 2 * kAttnRowsP + kAttnRowsP + pr];
      const float* src = a.part_o + (part * kAttnRowsP + pr) * 128 + d0;
      const float4_t o0 = *(const float4_t*)src, o1 = *(const float4_t*)(src + 4);
      const float mn = fmaxf(m, mp);
      const float sa = (m == -INFINITY) ? 0.f : exp2f(m - mn);
      const float sb = (mp == -INFINITY) ? 0.f : exp2f(mp - mn);
      lsum = lsum * sa + sb * lp;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        acc[j] = acc[j] * sa + sb * o0[j];
        acc[4 + j] = acc[4 + j] * sa + sb * o1[j];
      }
      m = mn;
    }
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] *= inv;
    const int tok = cb.tok0 + row / G, head = cb.kvh * G + row % G;
    store_out8(a.out, a.out_f16, ((size_t)(a.cu[cb.seq] + tok) * a.H + head) * kHeadDim + d0, acc,
               a.out_lo);
  }
}

// Zeroes rows [r0, r1) of a [T, width] activation: the inert pad rows.
__global__ void zero_rows_kernel(void* out, int f16, size_t start, size_t count, size_t lo) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  if (f16) ((half_t*)out)[start + i] = (half_t)0.f;
  else ((float*)out)[start + i] = 0.f;
  if (f16 == OUT_X2) ((half_t*)out)[lo + start + i] = (half_t)0.f;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

// Builds the work decomposition. Validates what the kernel relies on: every
// position a claimed row reads has a page-table entry inside the pool.
int attn_build_plan(int T, int B, const uint32_t* lengths, const uint32_t* extents,
                    const uint32_t* pages, int max_pages, int block, int capacity, int H,
                    int Hkv, AttnPlan& plan, int cascade_min, bool f32_q) {
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
  plan.seqlist.clear();
  plan.shared_positions = 0;
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
  // Positions per part of a context-split item (multiples of the 64-position
  // tile). Decode-style items stream: long parts amortize a workgroup's start
  // (page staging, first loads) and merge. Prefill-style items are MFMA-bound:
  // shorter parts spread a chunk's work over more workgroups. Both depend only
  // on the sequence itself, so a mixed launch decomposes every sequence as it
  // would alone. TGOHIP_ATTN_SPLIT / TGOHIP_ATTN_PSPLIT override them.
  // An override is capped so that a part's page-16 table always fits the
  // kMaxItemPages the kernel stages in LDS.
  static constexpr int kSplitCap = (kMaxItemPages - 4) * 16 / kAttnTile * kAttnTile;
  static const int split = [] {
    const char* e = getenv("TGOHIP_ATTN_SPLIT");
    const int v = std::min(e ? atoi(e) : kAttnSplitDecode, kSplitCap);
    return v >= kAttnTile ? v / kAttnTile * kAttnTile : kAttnSplitDecode;
  }();
  static const int psplit = [] {
    const char* e = getenv("TGOHIP_ATTN_PSPLIT");
    const int v = std::min(e ? atoi(e) : kAttnSplitPrefill, kSplitCap);
    return v >= kAttnTile ? v / kAttnTile * kAttnTile : kAttnSplitPrefill;
  }();
  // Shared prefixes (opt-in): decode sequences (one token) whose page rows
  // begin with the same pages attend to those positions together. A group's
  // prefix is the longest run of pages every member shares, cut to whole
  // 64-position tiles and to positions every member's token sees. Each batch
  // of up to 128/G members gets items over the prefix (split like prefill
  // items) writing partials; each member's own suffix is decode items writing
  // partials; the combine merges prefix parts, then suffix parts.
  std::vector<int> cpos(B, 0), cbase(B, 0), cnsp(B, 0), crow(B, 0);
  if (cascade_min >= 2) {
    std::vector<std::pair<uint32_t, int>> firsts;
    for (int s = 0; s < B; s++)
      if (extents[s] == 1 && G <= 16 && (int)lengths[s] >= kAttnTile)
        firsts.push_back({pages[(size_t)s * max_pages], s});
    std::stable_sort(firsts.begin(), firsts.end(),
                     [](const std::pair<uint32_t, int>& x, const std::pair<uint32_t, int>& y) {
                       return x.first < y.first;
                     });
    for (size_t i = 0; i < firsts.size();) {
      size_t j = i + 1;
      while (j < firsts.size() && firsts[j].first == firsts[i].first) j++;
      if ((int)(j - i) >= cascade_min) {
        const int lead = firsts[i].second;
        const uint32_t* lrow = pages + (size_t)lead * max_pages;
        int64_t ppos = lengths[lead];
        for (size_t k = i; k < j; k++) {
          const int sq = firsts[k].second;
          const uint32_t* row = pages + (size_t)sq * max_pages;
          const int64_t need = std::min<int64_t>((lengths[sq] + block - 1) / block,
                                                 (lengths[lead] + block - 1) / block);
          int64_t cp = 0;
          while (cp < need && row[cp] == lrow[cp]) cp++;
          ppos = std::min<int64_t>(ppos, std::min<int64_t>(cp * block, lengths[sq]));
        }
        ppos = ppos / kAttnTile * kAttnTile;
        if (ppos >= kAttnTile) {
          // Prefix parts are short: a group's few prefix items would otherwise
          // be the launch's longest chains.
          const int xsplit = std::min(psplit, kAttnSplitShared);
          const int per = std::max(1, kAttnRowsP / G);
          const int nsp = (int)((ppos + xsplit - 1) / xsplit);
          for (size_t b0 = i; b0 < j; b0 += per) {
            const int nb = (int)std::min<size_t>(per, j - b0);
            const int base = plan.parts;
            plan.parts += Hkv * nsp;
            const int off = (int)plan.seqlist.size();
            for (int k = 0; k < nb; k++) {
              const int sq = firsts[b0 + k].second;
              plan.seqlist.push_back(sq);
              cpos[sq] = (int)ppos;
              cbase[sq] = base;
              cnsp[sq] = nsp;
              crow[sq] = k * G;
            }
            for (int kvh = 0; kvh < Hkv; kvh++)
              for (int p = 0; p < nsp; p++)
                plan.items.push_back(AttnItem{lead, kvh, off, nb, p * xsplit,
                                              (int)std::min<int64_t>(ppos, (int64_t)(p + 1) * xsplit),
                                              base + kvh * nsp + p, 3});
          }
          plan.shared_positions += (int64_t)(j - i - 1) * ppos;
        }
      }
      i = j;
    }
  }
  // Leading pages a sequence shares with another (first page equal, then the
  // run of equal pages with the first sequence of that page): decode items
  // below that many positions use ordinary loads (kAttnSharedPages). The
  // cascade's suffix items start past its prefix.
  std::vector<int64_t> spos(B, 0);
  {
    std::vector<std::pair<uint32_t, int>> firsts;
    for (int s = 0; s < B; s++)
      if (extents[s] > 0 && lengths[s] > 0) firsts.push_back({pages[(size_t)s * max_pages], s});
    std::stable_sort(firsts.begin(), firsts.end(),
                     [](const std::pair<uint32_t, int>& x, const std::pair<uint32_t, int>& y) {
                       return x.first < y.first;
                     });
    for (size_t i = 0; i < firsts.size();) {
      size_t j = i + 1;
      while (j < firsts.size() && firsts[j].first == firsts[i].first) j++;
      if (j - i >= 2) {
        const int lead = firsts[i].second;
        const uint32_t* lrow = pages + (size_t)lead * max_pages;
        const int64_t lp = ((int64_t)lengths[lead] + block - 1) / block;
        int64_t lead_shared = 0;
        for (size_t k = i + 1; k < j; k++) {
          const int sq = firsts[k].second;
          const uint32_t* row = pages + (size_t)sq * max_pages;
          const int64_t need = std::min<int64_t>(((int64_t)lengths[sq] + block - 1) / block, lp);
          int64_t cp = 0;
          while (cp < need && row[cp] == lrow[cp]) cp++;
          spos[sq] = cp * block;
          lead_shared = std::max(lead_shared, cp * block);
        }
        spos[lead] = lead_shared;
      }
      i = j;
    }
  }
  auto dmode = [&](int s, int lo) { return lo < spos[s] ? kAttnSharedPages : 0; };
  for (int s = 0; s < B; s++) {
    const int n = (int)extents[s], L = (int)lengths[s];
    if (n == 0) continue;
    if (cpos[s] > 0) {
      // the suffix after the shared prefix, always as partials
      const int lo0 = cpos[s];
      const int splits = (L - lo0 + split - 1) / split;
      const int base = plan.parts;
      for (int p = 0; p < splits; p++) {
        const int lo = lo0 + p * split, hi = std::min(L, lo + split);
        for (int kvh = 0; kvh < Hkv; kvh++)
          plan.items.push_back(AttnItem{s, kvh, 0, n, lo, hi, base + kvh * splits + p, dmode(s, lo)});
      }
      for (int kvh = 0; kvh < Hkv; kvh++)
        plan.combines.push_back(AttnCombine{s, kvh, 0, n, base + kvh * splits, splits,
                                            cbase[s] + kvh * cnsp[s], cnsp[s], crow[s], 0});
      plan.parts += Hkv * splits;
      continue;
    }
    if (n * G <= 16) {
      // The kv heads of one part are adjacent in launch order: they read the
      // same 2 KiB position rows of the pool at about the same time.
      const int splits = (L + split - 1) / split;
      if (splits <= 1) {
        for (int kvh = 0; kvh < Hkv; kvh++)
          plan.items.push_back(AttnItem{s, kvh, 0, n, 0, L, -1, dmode(s, 0)});
      } else {
        const int base = plan.parts;
        for (int p = 0; p < splits; p++) {
          const int lo = p * split, hi = std::min(L, lo + split);
          for (int kvh = 0; kvh < Hkv; kvh++)
            plan.items.push_back(AttnItem{s, kvh, 0, n, lo, hi, base + kvh * splits + p, dmode(s, lo)});
        }
        for (int kvh = 0; kvh < Hkv; kvh++)
          plan.combines.push_back(AttnCombine{s, kvh, 0, n, base + kvh * splits, splits, -1, 0, 0, 0});
        plan.parts += Hkv * splits;
      }
    } else {
      // Prefill-style: 64 rows per item, and the context split into parts too,
      // so a long context is walked by many workgroups in parallel.
      const int tpi = std::max(1, kAttnRowsP / G);
      for (int t0 = 0; t0 < n; t0 += tpi) {
        const int nt = std::min(tpi, n - t0);
        const int hi = L - n + t0 + nt;
        const int splits = (hi + psplit - 1) / psplit;
        for (int kvh = 0; kvh < Hkv; kvh++) {
          if (splits <= 1) {
            plan.items.push_back(AttnItem{s, kvh, t0, nt, 0, hi, -1, 1});
          } else {
            const int part0 = plan.parts;
            for (int p = 0; p < splits; p++) {
              const int lo = p * psplit, h2 = std::min(hi, lo + psplit);
              plan.items.push_back(AttnItem{s, kvh, t0, nt, lo, h2, plan.parts++, 1});
            }
            plan.combines.push_back(AttnCombine{s, kvh, t0, nt, part0, splits, -1, 0, 0, 0});
          }
        }
      }
    }
  }
  // Launch order. Decode-style items stream K/V (HBM-bound); prefill-style
  // items re-read their sequence's K/V many times and are MFMA-bound. They are
  // interleaved evenly so both kinds run side by side for the whole launch,
  // each kind heavy-first so the tail is short items. Workgroup i is
  // dispatched to XCD i % 8, and the prefill items of one (sequence, kv head)
  // all re-read the same K/V stream: each stream is routed to one XCD (its
  // items take only that XCD's positions) so that XCD's L2 serves the
  // re-reads.
  {
    constexpr int kXcd = 8;
    std::vector<AttnItem> pre, dec;
    for (const AttnItem& x : plan.items) ((x.mode & kAttnModeMask) ? pre : dec).push_back(x);
    auto heavy = [](const AttnItem& x, const AttnItem& y) {
      return (x.kv_hi - x.kv_lo) > (y.kv_hi - y.kv_lo);
    };
    std::stable_sort(dec.begin(), dec.end(), heavy);
    // Decode items go heavy-first, which keeps the tail short, with f16 q.
    // With f32 q (tgo's arithmetic: two MFMAs per prefill product) decode
    // groups (the kv heads of one part) are taken alternately from the long
    // and the short end beside prefill items, so the heavier prefill MFMA
    // work meets a steady mix of streams: the C4 launch 0.218-0.220 ->
    // 0.209-0.212 ms (two alternating pairs of 40 steps). With f16 q and the
    // non-temporal decode loads heavy-first was 0.5% faster (5218-5283
    // against 5186-5228 tok/s, five alternating pairs of 60 steps).
    // TGOHIP_ATTN_ORDER (0 heavy-first, 1 alternating) overrides. The order
    // changes when items run, not what they compute.
    static const int order_env = [] { const char* e = getenv("TGOHIP_ATTN_ORDER"); return e ? atoi(e) : -1; }();
    const int order = order_env >= 0 ? order_env : (f32_q ? 1 : 0);
    if (order == 1 && !pre.empty() && !dec.empty()) {
      std::vector<std::pair<size_t, size_t>> grp;
      for (size_t i = 0; i < dec.size();) {
        size_t j = i + 1;
        while (j < dec.size() && dec[j].seq == dec[i].seq && dec[j].kv_lo == dec[i].kv_lo) j++;
        grp.push_back({i, j});
        i = j;
      }
      std::vector<AttnItem> alt;
      alt.reserve(dec.size());
      size_t lo = 0, hi = grp.size();
      bool front = true;
      while (lo < hi) {
        const auto g = front ? grp[lo++] : grp[--hi];
        for (size_t k = g.first; k < g.second; k++) alt.push_back(dec[k]);
        front = !front;
      }
      dec.swap(alt);
    }
    std::vector<std::vector<AttnItem>> q(kXcd);
    for (const AttnItem& x : pre) q[(x.seq * 131 + x.kvh) % kXcd].push_back(x);
    for (auto& qq : q) std::stable_sort(qq.begin(), qq.end(), heavy);
    const size_t total = pre.size() + dec.size();
    std::vector<AttnItem> out;
    out.reserve(total + kXcd * 4);
    std::vector<size_t> at(kXcd, 0);
    size_t taken_pre = 0, taken_dec = 0;
    while (taken_pre < pre.size() || taken_dec < dec.size()) {
      const int x = (int)(out.size() % kXcd);
      const bool pre_here = at[x] < q[x].size();
      // the prefill share of the launch so far stays at the overall share
      const bool want_pre = (double)(taken_pre + 1) * (double)total <=
                            (double)pre.size() * (double)(out.size() + 1) + 1e-9;
      if (pre_here && (want_pre || taken_dec == dec.size())) {
        out.push_back(q[x][at[x]++]);
        taken_pre++;
      } else if (taken_dec < dec.size()) {
        out.push_back(dec[taken_dec++]);
      } else {
        out.push_back(AttnItem{0, 0, 0, 0, 0, 0, -1, 2});  // this XCD's queue is empty
      }
    }
    while (!out.empty() && out.back().mode == 2) out.pop_back();
    plan.items.swap(out);
  }
  return 0;
}

int attn_enqueue(const AttnPlan& plan, const AttnDevPlan& dp, const void* q, int q_f16,
                 const void* k, const void* v, void* out, int out_form, int T, int H, int Hkv,
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
  a.seqlist = dp.seqlist;
  a.cu = dp.cu;
  a.lengths = dp.lengths;
  a.extents = dp.extents;
  a.pages = dp.pages;
  a.q_f16 = q_f16;
  a.out_f16 = out_form;
  a.out_lo = (size_t)T * H * kHeadDim;
  a.max_pages = max_pages;
  a.block = block;
  a.H = H;
  a.Hkv = Hkv;
  a.G = H / Hkv;
  a.qscale = scale * 1.4426950408889634f;
  if (!plan.items.empty()) {
    const dim3 grid((unsigned)plan.items.size());
    bool dec = true;
    for (const AttnItem& x : plan.items)
      dec = dec && ((x.mode & kAttnModeMask) == 0 || x.mode == 2);
    if (dec && block == 16 && q_f16) hipLaunchKernelGGL((attn_kernel<16, true, true>), grid, dim3(256), 0, stream, a);
    else if (dec && block == 16) hipLaunchKernelGGL((attn_kernel<16, false, true>), grid, dim3(256), 0, stream, a);
    else if (block == 16 && q_f16) hipLaunchKernelGGL((attn_kernel<16, true>), grid, dim3(256), 0, stream, a);
    else if (block == 16) hipLaunchKernelGGL((attn_kernel<16, false>), grid, dim3(256), 0, stream, a);
    else if (q_f16) hipLaunchKernelGGL((attn_kernel<0, true>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((attn_kernel<0, false>), grid, dim3(256), 0, stream, a);
  }
  if (!plan.combines.empty()) {
    // 16 rows per block: as many row blocks as the largest item needs (a
    // decode-only step's items have G rows: one block each, not eight)
    int rows = 1;
    for (const AttnCombine& x : plan.combines) rows = std::max(rows, x.ntok * H / Hkv);
    const unsigned ry = (unsigned)std::min((rows + 15) / 16, kAttnRowsP / 16);
    hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)plan.combines.size(), ry), dim3(256), 0,
                       stream, a);
  }
  if (plan.claimed < T) {
    const size_t start = (size_t)plan.claimed * H * kHeadDim;
    const size_t count = (size_t)(T - plan.claimed) * H * kHeadDim;
    hipLaunchKernelGGL(zero_rows_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0,
                       stream, out, out_form, start, count, a.out_lo);
  }
  TGOHIP_HIP(hipGetLastError());
  return 0;
}

}  // namespace tgohip
