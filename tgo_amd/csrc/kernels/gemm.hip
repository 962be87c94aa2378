// gemm.hip -- nn.Linear (nn/blocks.go:22-46): y[M,N] = x[M,K] . deq(W)[K,N] with
// the dequantization fused into the MFMA B operand, for every weight form tgo
// stores (nn/nn.go:118-136) plus the symmetric group-32-along-K int4 pack.
//
// Device weight layout ("fragment-major"), built once at upload by
// repack_kernel: for each block of 32 output columns (nb) and each 64-deep
// slice of K (ks), lane l of a wave owns column nb*32 + l%32 and, for substep
// j = 0..3, the eight k = ks*64 + 16j + 8*(l/32) + [0,8) -- exactly the B
// fragment of v_mfma_f32_32x32x16_f16. A wave therefore reads its weights with
// one contiguous 1 KiB (int4) / 2 KiB (int8) / 4 KiB (f16) burst per (nb, ks),
// dequantizes in registers and never stages weights through LDS.
//   int4: one u32 per substep; nibble slots hold k offsets 0,2,4,6,1,3,5,7 so
//         ((w >> 4j) & 0x000F000F) | 0x64006400 is the f16 pair (1024+q_2j,
//         1024+q_2j+1).
//   int8: two u32 per substep; bytes hold k offsets 0,2,1,3 as q+128 so the
//         0x00FF00FF mask yields consecutive-k f16 pairs (1024+b).
//   f16:  eight halves per substep.
// Dequantized value: round-to-nearest-even f16 of the exact (q - z) * s, which
// is computed with one exact packed subtraction and one rounded packed multiply.
//
// Tiling: waves side by side in N, each MW x 64 (MW/32 x 2 MFMA blocks of
// 32x32); a workgroup of 4 waves owns MW rows x 256 columns (gemm_pipe_kernel
// also runs 8 waves over 512 columns, which halves the activation tile's
// reads per column). The activation tile (MW x 64 f16) is staged in LDS,
// XOR-swizzled: double-buffered through registers in gemm_kernel, a
// four-stage ring filled by LDS DMA in gemm_pipe_kernel. An f32 activation is carried as f16 hi + lo (two MFMAs) so
// the product keeps ~22 bits of the activation. Split-K over grid.z writes f32
// partials that a reduction kernel (or the consumer) sums in split order
// (deterministic).
#include "../common.h"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace tgohip {

struct GemmArgs {
  const void* x;        // [M,K] f16 or f32 (or the hi plane of an XK_X2 pair)
  const void* xlo;      // XK_X2: the lo plane [M,K] f16; null otherwise
  const void* wp;       // packed payload
  const half_t* ws;     // packed scales (form dependent)
  const half_t* wz;     // packed zero+1024 (I4_TGO only)
  void* y;              // output (EPI dependent)
  float* part;          // split-K partials: split s at part + s * pstride, [M][N]
  size_t pstride;
  int M, K, N;
  int ksteps_per_split;
};

__device__ __forceinline__ half2_t as_h2(uint32_t u) {
  union { uint32_t u; half2_t h; } c;
  c.u = u;
  return c.h;
}

// ---- dequantization of one substep's B fragment (8 consecutive k) ----------
__device__ __forceinline__ half8_t deq_i4_sym(uint32_t w, half_t s) {
  const half2_t sp = {s, s};
  // A nibble in bits 0-3 of a 16-bit half merged into 0x6400 (1024.0) reads
  // as 1024 + q; one in bits 4-7 merged into 0x5400 (64.0, whose mantissa bit
  // 4 is worth 1) reads as 64 + q. Subtracting 1032 or 72 leaves q - 8
  // exactly, so substeps 0/1 come from w and 2/3 from w >> 8 with one shift.
  // The masks sit in registers so each mask-and-merge is one v_and_or_b32
  // (its encoding takes no literal constants).
  uint32_t m0 = 0x000F000Fu, m1 = 0x00F000F0u, g0 = 0x64006400u, g1 = 0x54005400u;
  asm("" : "+v"(m0), "+v"(m1), "+v"(g0), "+v"(g1));
  const half2_t b0 = {(half_t)1032.f, (half_t)1032.f}, b1 = {(half_t)72.f, (half_t)72.f};
  const uint32_t w8 = w >> 8;
  const half2_t h[4] = {(as_h2((w & m0) | g0) - b0) * sp, (as_h2((w & m1) | g1) - b1) * sp,
                        (as_h2((w8 & m0) | g0) - b0) * sp, (as_h2((w8 & m1) | g1) - b1) * sp};
  half8_t o;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    o[2 * j] = h[j][0];
    o[2 * j + 1] = h[j][1];
  }
  return o;
}
// The codes q - 8 of one substep's B fragment, unscaled: small integers, exact
// in f16 (the masks and merge constants of deq_i4_sym).
__device__ __forceinline__ half8_t i4_sym_codes(uint32_t w) {
  uint32_t m0 = 0x000F000Fu, m1 = 0x00F000F0u, g0 = 0x64006400u, g1 = 0x54005400u;
  asm("" : "+v"(m0), "+v"(m1), "+v"(g0), "+v"(g1));
  const half2_t b0 = {(half_t)1032.f, (half_t)1032.f}, b1 = {(half_t)72.f, (half_t)72.f};
  const uint32_t w8 = w >> 8;
  const half2_t h[4] = {as_h2((w & m0) | g0) - b0, as_h2((w & m1) | g1) - b1,
                        as_h2((w8 & m0) | g0) - b0, as_h2((w8 & m1) | g1) - b1};
  half8_t o;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    o[2 * j] = h[j][0];
    o[2 * j + 1] = h[j][1];
  }
  return o;
}
__device__ __forceinline__ half8_t deq_i4_asym(uint32_t w, half8_t s, half8_t zz) {
  half8_t o;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    half2_t h = as_h2(((w >> (4 * j)) & 0x000F000Fu) | 0x64006400u);
    const half2_t z2 = {zz[2 * j], zz[2 * j + 1]};
    const half2_t s2 = {s[2 * j], s[2 * j + 1]};
    h = h - z2;
    h = h * s2;
    o[2 * j] = h[0];
    o[2 * j + 1] = h[1];
  }
  return o;
}
__device__ __forceinline__ half8_t deq_i8(uint32_t w0, uint32_t w1, half8_t s) {
  const half2_t bias = {(half_t)1152.f, (half_t)1152.f};
  half8_t o;
  const uint32_t ws[2] = {w0, w1};
#pragma unroll
  for (int u = 0; u < 2; u++) {
    half2_t lo = as_h2((ws[u] & 0x00FF00FFu) | 0x64006400u);
    half2_t hi = as_h2(((ws[u] >> 8) & 0x00FF00FFu) | 0x64006400u);
    const half2_t s0 = {s[4 * u], s[4 * u + 1]}, s1 = {s[4 * u + 2], s[4 * u + 3]};
    lo = (lo - bias) * s0;
    hi = (hi - bias) * s1;
    o[4 * u] = lo[0];
    o[4 * u + 1] = lo[1];
    o[4 * u + 2] = hi[0];
    o[4 * u + 3] = hi[1];
  }
  return o;
}

// The lane's raw material for one (nb, ks): payload plus the scales it needs,
// sized per form so no register is spent on another form's fields.
template <int FORM> struct BRaw;
template <> struct BRaw<TGOHIP_FORM_F16> { uint4 p[4]; };
template <> struct BRaw<TGOHIP_FORM_I8> { uint4 p[2]; uint4 s[4]; };
template <> struct BRaw<TGOHIP_FORM_I4_TGO> { uint4 p; uint4 s[4]; uint4 z[4]; };
template <> struct BRaw<TGOHIP_FORM_I4_SYM> { uint4 p; uint32_t s; };

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// A 16-byte weight load; NT: non-temporal (the nt bit), for a launch that
// reads each weight once. The small-M kernel's int4 gate/up at one row went
// from 15.6 to 13.5 us with it, the LM head from 70.7 to 64.8; the pipelined
// kernel's row tiles share weights through L2, and nt loads made its 64- and
// 128-row down 12-18% slower.
template <bool NT>
__device__ __forceinline__ uint4 ldw16(const void* p) {
  if constexpr (NT) {
    const u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *(const uint4*)p;
  }
}

template <bool NT = false>
__device__ __forceinline__ void load_braw(const GemmArgs& g, int nb, int ks, int lane,
                                          BRaw<TGOHIP_FORM_F16>& r) {
  const size_t slot = ((size_t)nb * (g.K / 64) + ks) * 64 + lane;
  const uint4* pp = (const uint4*)((const char*)g.wp + slot * 64);
#pragma unroll
  for (int i = 0; i < 4; i++) r.p[i] = ldw16<NT>(pp + i);
}
template <bool NT = false>
__device__ __forceinline__ void load_braw(const GemmArgs& g, int nb, int ks, int lane,
                                          BRaw<TGOHIP_FORM_I8>& r) {
  const int KS = g.K / 64;
  const size_t slot = ((size_t)nb * KS + ks) * 64 + lane;
  const uint4* pp = (const uint4*)((const char*)g.wp + slot * 32);
  r.p[0] = ldw16<NT>(pp);
  r.p[1] = ldw16<NT>(pp + 1);
  const int h = lane >> 5;
#pragma unroll
  for (int j = 0; j < 4; j++) r.s[j] = *(const uint4*)(g.ws + ((((size_t)nb * KS + ks) * 4 + j) * 2 + h) * 8);
}
template <bool NT = false>
__device__ __forceinline__ void load_braw(const GemmArgs& g, int nb, int ks, int lane,
                                          BRaw<TGOHIP_FORM_I4_TGO>& r) {
  const int KS = g.K / 64;
  const size_t slot = ((size_t)nb * KS + ks) * 64 + lane;
  r.p = ldw16<NT>((const char*)g.wp + slot * 16);
  const int h = lane >> 5;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const size_t o = ((((size_t)nb * KS + ks) * 4 + j) * 2 + h) * 8;
    r.s[j] = *(const uint4*)(g.ws + o);
    r.z[j] = *(const uint4*)(g.wz + o);
  }
}
template <bool NT = false>
__device__ __forceinline__ void load_braw(const GemmArgs& g, int nb, int ks, int lane,
                                          BRaw<TGOHIP_FORM_I4_SYM>& r) {
  // (nb, ks) is uniform across the wave: a scalar base plus a 32-bit lane
  // offset, so the loads need no 64-bit vector address arithmetic.
  const size_t blk = (size_t)nb * (g.K / 64) + ks;
  r.p = ldw16<NT>((const char*)g.wp + blk * 1024 + (uint32_t)lane * 16u);
  r.s = *(const uint32_t*)((const char*)g.ws + blk * 128 + (uint32_t)(lane & 31) * 4u);
}

__device__ __forceinline__ uint32_t word_of(const uint4& p, int j) {
  return j == 0 ? p.x : j == 1 ? p.y : j == 2 ? p.z : p.w;
}

union U16B { uint4 u; half8_t h; };

__device__ __forceinline__ half8_t bfrag(const BRaw<TGOHIP_FORM_F16>& r, int j) {
  U16B c;
  c.u = r.p[j];
  return c.h;
}
__device__ __forceinline__ half8_t bfrag(const BRaw<TGOHIP_FORM_I4_SYM>& r, int j) {
  union { uint32_t u; half2_t h; } sc;
  sc.u = r.s;
  return deq_i4_sym(word_of(r.p, j), j < 2 ? sc.h[0] : sc.h[1]);
}
__device__ __forceinline__ half8_t bfrag(const BRaw<TGOHIP_FORM_I4_TGO>& r, int j) {
  U16B s, z;
  s.u = r.s[j];
  z.u = r.z[j];
  return deq_i4_asym(word_of(r.p, j), s.h, z.h);
}
__device__ __forceinline__ half8_t bfrag(const BRaw<TGOHIP_FORM_I8>& r, int j) {
  const uint4 q = r.p[j >> 1];
  const uint32_t w0 = (j & 1) ? q.z : q.x, w1 = (j & 1) ? q.w : q.y;
  U16B s;
  s.u = r.s[j];
  return deq_i8(w0, w1, s.h);
}

// ---- exact dequantized weights as two f16 fragments ------------------------
// hi = RNE_f16((q - z) * s) and lo = (q - z) * s - hi, each f16, so hi + lo is
// the exact product tgo's CPU path multiplies (the f32 dequantization): (q - z)
// has at most 8 significant bits and s 11, so the residual after hi's 11 bits
// fits lo's (down to f16's subnormal spacing, 2^-24). lo comes from one fused
// multiply-add, q*s - hi, rounded once and exact. An MFMA with each half gives
// the product against the unrounded weight.
__device__ __forceinline__ void split_pair(half2_t d, half2_t s2, half2_t& hi, half2_t& lo) {
  hi = d * s2;
  lo = __builtin_elementwise_fma(d, s2, -hi);
}
__device__ __forceinline__ void pack_pair(half8_t& o, int j, half2_t h) {
  o[2 * j] = h[0];
  o[2 * j + 1] = h[1];
}
template <int FORM>
__device__ __forceinline__ void bfrag_split(const BRaw<FORM>& r, int j, half8_t& hi, half8_t& lo);
template <>
__device__ __forceinline__ void bfrag_split(const BRaw<TGOHIP_FORM_I4_SYM>& r, int j, half8_t& hi,
                                            half8_t& lo) {
  union { uint32_t u; half2_t h; } sc;
  sc.u = r.s;
  const half_t s = j < 2 ? sc.h[0] : sc.h[1];
  const half2_t sp = {s, s};
  const uint32_t w = word_of(r.p, j), w8 = w >> 8;
  const half2_t b0 = {(half_t)1032.f, (half_t)1032.f}, b1 = {(half_t)72.f, (half_t)72.f};
  // q - 8 exactly, as in deq_i4_sym (masks in registers: one v_and_or_b32 each)
  uint32_t m0 = 0x000F000Fu, m1 = 0x00F000F0u, g0 = 0x64006400u, g1 = 0x54005400u;
  asm("" : "+v"(m0), "+v"(m1), "+v"(g0), "+v"(g1));
  const half2_t d[4] = {as_h2((w & m0) | g0) - b0, as_h2((w & m1) | g1) - b1,
                        as_h2((w8 & m0) | g0) - b0, as_h2((w8 & m1) | g1) - b1};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    half2_t h, l;
    split_pair(d[i], sp, h, l);
    pack_pair(hi, i, h);
    pack_pair(lo, i, l);
  }
}
template <>
__device__ __forceinline__ void bfrag_split(const BRaw<TGOHIP_FORM_I4_TGO>& r, int j, half8_t& hi,
                                            half8_t& lo) {
  U16B s, z;
  s.u = r.s[j];
  z.u = r.z[j];
  const uint32_t w = word_of(r.p, j);
  uint32_t m0 = 0x000F000Fu, g0 = 0x64006400u;
  asm("" : "+v"(m0), "+v"(g0));
#pragma unroll
  for (int i = 0; i < 4; i++) {
    // (1024 + q) - (1024 + z) = q - z exactly
    const half2_t d = as_h2(((w >> (4 * i)) & m0) | g0) - half2_t{z.h[2 * i], z.h[2 * i + 1]};
    half2_t h, l;
    split_pair(d, half2_t{s.h[2 * i], s.h[2 * i + 1]}, h, l);
    pack_pair(hi, i, h);
    pack_pair(lo, i, l);
  }
}
template <>
__device__ __forceinline__ void bfrag_split(const BRaw<TGOHIP_FORM_I8>& r, int j, half8_t& hi,
                                            half8_t& lo) {
  const uint4 q = r.p[j >> 1];
  const uint32_t ws[2] = {(j & 1) ? q.z : q.x, (j & 1) ? q.w : q.y};
  U16B s;
  s.u = r.s[j];
  const half2_t bias = {(half_t)1152.f, (half_t)1152.f};
  uint32_t m0 = 0x00FF00FFu, g0 = 0x64006400u;
  asm("" : "+v"(m0), "+v"(g0));
#pragma unroll
  for (int u = 0; u < 2; u++) {
    // (1024 + q + 128) - 1152 = q exactly
    const half2_t dl = as_h2((ws[u] & m0) | g0) - bias;
    const half2_t dh = as_h2(((ws[u] >> 8) & m0) | g0) - bias;
    half2_t h, l;
    split_pair(dl, half2_t{s.h[4 * u], s.h[4 * u + 1]}, h, l);
    pack_pair(hi, 2 * u, h);
    pack_pair(lo, 2 * u, l);
    split_pair(dh, half2_t{s.h[4 * u + 2], s.h[4 * u + 3]}, h, l);
    pack_pair(hi, 2 * u + 1, h);
    pack_pair(lo, 2 * u + 1, l);
  }
}
template <>
__device__ __forceinline__ void bfrag_split(const BRaw<TGOHIP_FORM_F16>& r, int j, half8_t& hi,
                                            half8_t& lo) {
  hi = bfrag(r, j);  // f16 weights are exact as stored
  lo = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
}

// silu(g) = g / (1 + e^-g) (nn/blocks.go:62-66) with the hardware reciprocal
// (v_rcp_f32, 1 ulp) in place of the IEEE division's ten-instruction sequence:
// the SwiGLU epilogue of the C4 gate/up 209 -> 205 us.
__device__ __forceinline__ float silu_f(float g) { return g * __builtin_amdgcn_rcpf(1.f + __expf(-g)); }

// 16-byte slot of (row, k-chunk) in an LDS activation tile of 8 chunks per row.
// The XOR with (row/2) % 8 spreads any 16 consecutive rows of one k-chunk over
// all 64 banks (a bank row is 256 bytes = two tile rows), so the MFMA operand
// reads (16 lanes = 16 rows per LDS cycle) and the row-wise stores are
// conflict-free.
__device__ __forceinline__ int a_slot(int row, int kc) { return row * 8 + (kc ^ ((row >> 1) & 7)); }

// One SwiGLU output at element o of [M, N/2]: f16, f32, or the f16 hi plane
// and the lo plane (f16(v - hi)) M*N/2 elements after it (the activation pair
// the exact down projection reads).
template <int EPI>
__device__ __forceinline__ void store_swiglu(const GemmArgs& g, size_t o, float v) {
  if (EPI == EPI_SWIGLU_F32) {
    ((float*)g.y)[o] = v;
  } else {
    const half_t h = (half_t)v;
    ((half_t*)g.y)[o] = h;
    if (EPI == EPI_SWIGLU_X2) ((half_t*)g.y)[(size_t)g.M * (g.N / 2) + o] = (half_t)(v - (float)h);
  }
}

// Epilogue shared by the GEMM kernels. Lane holds D[8*(r/4) + 4*h + (r%4)][c32]
// of each 32x32 block; a split-K launch writes f32 partials for its split.
template <int EPI, int MB>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& g, const float16_t (&acc)[MB][2],
                                              int m0, int nbw0, const bool (&nbv)[2], int h,
                                              int c32, bool split, int z) {
#pragma unroll
  for (int mb = 0; mb < MB; mb++) {
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int row = m0 + mb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
      if (row >= g.M) continue;
      if (split) {
        float* dst = g.part + (size_t)z * g.pstride + (size_t)row * g.N;
#pragma unroll
        for (int b = 0; b < 2; b++)
          if (nbv[b]) dst[(nbw0 + b) * 32 + c32] = acc[mb][b][r];
      } else if (EPI == EPI_SWIGLU_F16 || EPI == EPI_SWIGLU_F32 || EPI == EPI_SWIGLU_X2) {
        if (nbv[1]) {
          const float v = silu_f(acc[mb][0][r]) * acc[mb][1][r];
          const int col = (nbw0 >> 1) * 32 + c32;
          const size_t o = (size_t)row * (g.N / 2) + col;
          store_swiglu<EPI>(g, o, v);
        }
      } else {
#pragma unroll
        for (int b = 0; b < 2; b++) {
          if (!nbv[b]) continue;
          const size_t o = (size_t)row * g.N + (nbw0 + b) * 32 + c32;
          if (EPI == EPI_F32) ((float*)g.y)[o] = acc[mb][b][r];
          else if (EPI == EPI_F16) ((half_t*)g.y)[o] = (half_t)acc[mb][b][r];
          else ((float*)g.y)[o] += acc[mb][b][r];
        }
      }
    }
  }
}

// A workgroup barrier that orders LDS only: global loads in flight stay in
// flight across it (__syncthreads would wait for them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ASPLIT (f32 activations, tgo's arithmetic): the activation is carried as f16
// hi + lo (about 22 bits) and the quantized weights as their exact hi + lo
// (bfrag_split), three MFMAs per product (hi.hi, lo.hi, hi.lo; lo.lo is below
// f32 rounding): the product of the f32 activation and the unrounded
// dequantized weight, f32 accumulated, as tgo's CPU path computes it.
template <int FORM, int MW, bool ASPLIT, int EPI>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmArgs g) {
  constexpr int MB = MW / 32;
  constexpr int APLANES = ASPLIT ? 2 : 1;
  constexpr bool BSPLIT = ASPLIT && FORM != TGOHIP_FORM_F16;
  __shared__ __attribute__((aligned(16))) half_t As[2][APLANES][MW * 64];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, c32 = lane & 31;
  const int NBT = g.N / 32;
  const int nbw0 = blockIdx.x * 8 + wave * 2;
  const int m0 = blockIdx.y * MW;
  const int KS = g.K / 64;
  const int ks0 = blockIdx.z * g.ksteps_per_split;
  const int ks1 = min(KS, ks0 + g.ksteps_per_split);
  const bool nbv[2] = {nbw0 < NBT, nbw0 + 1 < NBT};

  // A tile loader: MW rows x 64 k. Each thread moves (MW*64)/256 = MW/4
  // elements as chunks of 8.
  constexpr int ACH = MW / 32;  // chunks of 8 elements per thread
  uint4 areg[ACH][APLANES];
  auto load_a = [&](int ks) {
#pragma unroll
    for (int i = 0; i < ACH; i++) {
      const int c = tid + 256 * i, row = c >> 3, kc = c & 7;
      const int gm = m0 + row;
      if (gm < g.M) {
        const size_t off = (size_t)gm * g.K + ks * 64 + kc * 8;
        if (ASPLIT && g.xlo) {
          // an XK_X2 pair: hi and lo as their producer split them
          areg[i][0] = *(const uint4*)((const half_t*)g.x + off);
          areg[i][APLANES - 1] = *(const uint4*)((const half_t*)g.xlo + off);
        } else if (ASPLIT) {
          const float4_t u = *(const float4_t*)((const float*)g.x + off);
          const float4_t w = *(const float4_t*)((const float*)g.x + off + 4);
          const float v[8] = {u[0], u[1], u[2], u[3], w[0], w[1], w[2], w[3]};
          union { uint4 u; half8_t h; } hi, lo;
#pragma unroll
          for (int e = 0; e < 8; e++) {
            const half_t hv = (half_t)v[e];
            hi.h[e] = hv;
            lo.h[e] = (half_t)(v[e] - (float)hv);
          }
          areg[i][0] = hi.u;
          if (APLANES > 1) areg[i][APLANES - 1] = lo.u;
        } else {
          areg[i][0] = *(const uint4*)((const half_t*)g.x + off);
        }
      } else {
#pragma unroll
        for (int p = 0; p < APLANES; p++) areg[i][p] = make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < ACH; i++) {
      const int c = tid + 256 * i, row = c >> 3, kc = c & 7;
      const int phys = a_slot(row, kc);
#pragma unroll
      for (int p = 0; p < APLANES; p++) ((uint4*)As[buf][p])[phys] = areg[i][p];
    }
  };

  float16_t acc[MB][2];
#pragma unroll
  for (int mb = 0; mb < MB; mb++)
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mb][b][r] = 0.f;

  BRaw<FORM> bcur[2], bnext[2];
  if (ks0 < ks1) {
    load_a(ks0);
#pragma unroll
    for (int b = 0; b < 2; b++)
      if (nbv[b]) load_braw(g, nbw0 + b, ks0, lane, bcur[b]);
    store_a(0);
  }
  lds_barrier();
  int buf = 0;
  for (int ks = ks0; ks < ks1; ks++) {
    const bool more = ks + 1 < ks1;
    if (more) {
      load_a(ks + 1);
#pragma unroll
      for (int b = 0; b < 2; b++)
        if (nbv[b]) load_braw(g, nbw0 + b, ks + 1, lane, bnext[b]);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      half8_t bf[2], bl[2];
#pragma unroll
      for (int b = 0; b < 2; b++) {
        if constexpr (BSPLIT) bfrag_split(bcur[b], j, bf[b], bl[b]);
        else bf[b] = bfrag(bcur[b], j);
      }
#pragma unroll
      for (int mb = 0; mb < MB; mb++) {
        const int row = mb * 32 + c32;
        const int kc = 2 * j + h;
        const int phys = a_slot(row, kc);
#pragma unroll
        for (int p = 0; p < APLANES; p++) {
          const half8_t af = ((const half8_t*)As[buf][p])[phys];
#pragma unroll
          for (int b = 0; b < 2; b++) {
            acc[mb][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[b], acc[mb][b], 0, 0, 0);
            if (BSPLIT && p == 0)
              acc[mb][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bl[b], acc[mb][b], 0, 0, 0);
          }
        }
      }
    }
    if (more) store_a(buf ^ 1);
    lds_barrier();
    buf ^= 1;
    if (more) {
#pragma unroll
      for (int b = 0; b < 2; b++) bcur[b] = bnext[b];
    }
  }

  gemm_epilogue<EPI, MB>(g, acc, m0, nbw0, nbv, h, c32, gridDim.z > 1, blockIdx.z);
}

// Pipelined variant for f16 activations at larger M (the prefill-sized
// projections). B fragments (the weight stream) for k-step j are issued at
// step j-2 into a register ring; A (128 rows x 64 k of f16
// activations, mostly L2-resident) is issued at step j-1 and written to a
// double-buffered LDS tile at the end of that step. Barriers order LDS only, so
// loads stay in flight across them.
// ---- the pipelined kernel's B operand per form ------------------------------
// The register part of one (column block, k-step) of B. For int8 and tgo's
// int4 the per-k scales (and zeros) are the same for the 32 columns of a
// block, so they travel by LDS DMA with the activation tile instead of in
// registers (8 scale/zero pairs per lane per substep would not fit).
template <int FORM> struct PipeB;
template <> struct PipeB<TGOHIP_FORM_I4_SYM> { uint4 p; uint32_t s; };
template <> struct PipeB<TGOHIP_FORM_I4_TGO> { uint4 p; };
template <> struct PipeB<TGOHIP_FORM_I8> { uint4 p[2]; };

template <int FORM> constexpr bool pipe_lds_scales() { return FORM != TGOHIP_FORM_I4_SYM; }
// Vector memory instructions a wave issues per k-step for its two B blocks.
template <int FORM> constexpr int pipe_b_loads() { return FORM == TGOHIP_FORM_I4_TGO ? 2 : 4; }

__device__ __forceinline__ void load_pipeb(const GemmArgs& g, int nb, int ks, int lane,
                                           PipeB<TGOHIP_FORM_I4_SYM>& r) {
  BRaw<TGOHIP_FORM_I4_SYM> b;
  load_braw(g, nb, ks, lane, b);
  r.p = b.p;
  r.s = b.s;
}
__device__ __forceinline__ void load_pipeb(const GemmArgs& g, int nb, int ks, int lane,
                                           PipeB<TGOHIP_FORM_I4_TGO>& r) {
  const size_t blk = (size_t)nb * (g.K / 64) + ks;
  r.p = *(const uint4*)((const char*)g.wp + blk * 1024 + (uint32_t)lane * 16u);
}
__device__ __forceinline__ void load_pipeb(const GemmArgs& g, int nb, int ks, int lane,
                                           PipeB<TGOHIP_FORM_I8>& r) {
  const size_t blk = (size_t)nb * (g.K / 64) + ks;
  const uint4* pp = (const uint4*)((const char*)g.wp + blk * 2048 + (uint32_t)lane * 32u);
  r.p[0] = pp[0];
  r.p[1] = pp[1];
}
// Substep j's B fragment. sz: this wave's scale region of the k-step's stage
// (scales of block b at b*64 + (2j + h)*8, zeros 128 halves further).
__device__ __forceinline__ half8_t pipe_bfrag(const PipeB<TGOHIP_FORM_I4_SYM>& r, int j,
                                              const half_t*, int, int) {
  BRaw<TGOHIP_FORM_I4_SYM> x;
  x.p = r.p;
  x.s = r.s;
  return bfrag(x, j);
}
__device__ __forceinline__ half8_t pipe_bfrag(const PipeB<TGOHIP_FORM_I4_TGO>& r, int j,
                                              const half_t* sz, int b, int h) {
  const half8_t s8 = *(const half8_t*)(sz + b * 64 + (2 * j + h) * 8);
  const half8_t z8 = *(const half8_t*)(sz + 128 + b * 64 + (2 * j + h) * 8);
  return deq_i4_asym(word_of(r.p, j), s8, z8);
}
__device__ __forceinline__ half8_t pipe_bfrag(const PipeB<TGOHIP_FORM_I8>& r, int j,
                                              const half_t* sz, int b, int h) {
  const half8_t s8 = *(const half8_t*)(sz + b * 64 + (2 * j + h) * 8);
  const uint4 q = r.p[j >> 1];
  return deq_i8((j & 1) ? q.z : q.x, (j & 1) ? q.w : q.y, s8);
}

// Substep j's B fragment as the exact hi + lo pair (bfrag_split).
__device__ __forceinline__ void pipe_bfrag_x(const PipeB<TGOHIP_FORM_I4_SYM>& r, int j,
                                             const half_t*, int, int, half8_t& hi, half8_t& lo) {
  BRaw<TGOHIP_FORM_I4_SYM> x;
  x.p = r.p;
  x.s = r.s;
  bfrag_split(x, j, hi, lo);
}
__device__ __forceinline__ void pipe_bfrag_x(const PipeB<TGOHIP_FORM_I4_TGO>& r, int j,
                                             const half_t* sz, int b, int h, half8_t& hi,
                                             half8_t& lo) {
  BRaw<TGOHIP_FORM_I4_TGO> x;
  x.p = r.p;
  U16B sv, zv;
  sv.h = *(const half8_t*)(sz + b * 64 + (2 * j + h) * 8);
  zv.h = *(const half8_t*)(sz + 128 + b * 64 + (2 * j + h) * 8);
  x.s[j] = sv.u;
  x.z[j] = zv.u;
  bfrag_split(x, j, hi, lo);
}
__device__ __forceinline__ void pipe_bfrag_x(const PipeB<TGOHIP_FORM_I8>& r, int j,
                                             const half_t* sz, int b, int h, half8_t& hi,
                                             half8_t& lo) {
  BRaw<TGOHIP_FORM_I8> x;
  x.p[0] = r.p[0];
  x.p[1] = r.p[1];
  U16B sv;
  sv.h = *(const half8_t*)(sz + b * 64 + (2 * j + h) * 8);
  x.s[j] = sv.u;
  bfrag_split(x, j, hi, lo);
}

// NW waves (4 or 8) side by side in N: a workgroup owns MW rows x 64*NW
// columns. With KQ = 2 the workgroup holds two such groups of NW waves, each
// over one half of the workgroup's k-steps with its own A ring, and group 1
// hands its sums to group 0 through LDS at the end (acc0 + acc1, a fixed
// order): two waves per SIMD where the tiles alone would give one.
// EX (tgo's f32 arithmetic, XK_X2 activations): the A tile is the activation
// pair, hi and lo planes DMA'd side by side into each stage, and the weights
// the exact hi + lo pair (pipe_bfrag_x): three MFMAs per product (hi.hi,
// lo.hi, hi.lo), the f32 activation times the unrounded dequantized weight.
// Symmetric int4 (one scale per 32 k of a column) factors instead:
// sum_k x w = sum_g s_g (sum_{k in g} x q), and the codes q are exact f16, so
// each group's inner sum is two MFMAs (x_hi.q, x_lo.q) into a group
// accumulator that one f32 fma per output then scales into the sum. Every
// product x_hi q, x_lo q is exact and s_g multiplies in f32, so this is
// tgo's f32 dequantize-then-dot up to f32 rounding order, with the lo.lo term
// (2^-22 relative) dropped as in the three-MFMA form.
template <int FORM, int EPI, int MW, int NW, int KQ = 1, bool EX = false>
__global__ __launch_bounds__((64 * NW * KQ), (8 / (NW * KQ))) void gemm_pipe_kernel(
    GemmArgs g, int tiles_n, int tiles, int colmajor, int xsplit, QKRopeArgs qa) {
  constexpr int MB = MW / 32;
  constexpr bool FX = EX && FORM == TGOHIP_FORM_I4_SYM;  // factored scales
  constexpr int ACH = MW / (8 * NW);  // 1 KiB LDS-DMA chunks per wave per k-step and plane
  constexpr int AP = EX ? 2 : 1;      // activation planes per stage
  static_assert(KQ == 1 || (KQ == 2 && NW * MW * 256 <= 4 * 2 * MW * 128),
                "group 1's sums fit in the A ring");
  // Four LDS stages, separate arrays so the compiler can tell a DMA into one
  // stage from reads of another; group q's tile at q * AP * MW * 64 of each
  // (with EX its lo plane MW * 64 halves after its hi plane).
  __shared__ __attribute__((aligned(16))) half_t As0[KQ * AP * MW * 64];
  __shared__ __attribute__((aligned(16))) half_t As1[KQ * AP * MW * 64];
  __shared__ __attribute__((aligned(16))) half_t As2[KQ * AP * MW * 64];
  __shared__ __attribute__((aligned(16))) half_t As3[KQ * AP * MW * 64];
  half_t* const As[4] = {As0, As1, As2, As3};
  // Per-stage scales and zeros of the waves' column blocks (int8, tgo int4).
  constexpr bool LS = pipe_lds_scales<FORM>();
  constexpr int SZN = LS ? NW * 256 : 8;
  __shared__ __attribute__((aligned(16))) half_t Sz0[KQ * SZN];
  __shared__ __attribute__((aligned(16))) half_t Sz1[KQ * SZN];
  __shared__ __attribute__((aligned(16))) half_t Sz2[KQ * SZN];
  __shared__ __attribute__((aligned(16))) half_t Sz3[KQ * SZN];
  half_t* const Sz[4] = {Sz0, Sz1, Sz2, Sz3};

  // XCD x (workgroup b runs on XCD b % 8) owns the column tiles c = x (mod 8):
  // each weight column tile is streamed into one XCD's L2 and serves every row
  // tile there. Within an XCD the order is row-major over its columns (the
  // workgroups in flight share a row tile of activations), or with colmajor
  // column-major (they share a column tile of weights: its row tiles run side
  // by side and read it from HBM once). With xsplit (2, 4 or 8) split-K
  // slices the XCDs instead of riding grid.z: XCD x takes split x / G
  // (G = 8 / xsplit) and, of that split, the column tiles c = x % G (mod G),
  // so each XCD reads only its split's share of the activations (with 8
  // splits a 128-row step's activations cross into the L2s once, not 8 times).
  const int x = (int)(blockIdx.x & 7), j = (int)(blockIdx.x >> 3);
  int G = 8, r = x, split = (int)blockIdx.z, nsplit = (int)gridDim.z;
  if (xsplit > 1) {
    G = 8 / xsplit;
    split = x / G;
    r = x - split * G;
    nsplit = xsplit;
  }
  const int cols_x = (tiles_n - r + G - 1) / G;
  const int rows_t = tiles / tiles_n;
  if (cols_x <= 0 || j >= cols_x * rows_t) return;
  int tm, tn;
  if (colmajor) {
    const int cj = j / rows_t;
    tm = j - cj * rows_t;
    tn = r + G * cj;
  } else {
    tm = j / cols_x;
    tn = r + G * (j - tm * cols_x);
  }

  const int tid = threadIdx.x, lane = tid & 63;
  const int wq = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
  const int wave = wq % NW, kq = wq / NW;  // column wave, k group
  const int h = lane >> 5, c32 = lane & 31;
  const int NBT = g.N / 32;
  const int nbw0 = tn * 2 * NW + wave * 2;
  const int m0 = tm * MW;
  const int KS = g.K / 64;
  // k group q takes the q-th 1/KQ of the workgroup's k-steps (the host makes
  // each a multiple of 4)
  const int nkw = min(KS, split * g.ksteps_per_split + g.ksteps_per_split) - split * g.ksteps_per_split;
  const int nk = nkw / KQ;
  const int ks0 = split * g.ksteps_per_split + kq * nk;
  const int aq = kq * AP * MW * 64, sq = kq * SZN;  // the group's offsets in each A and scale stage
  const bool nbv[2] = {nbw0 < NBT, nbw0 + 1 < NBT};
  // Out-of-range column blocks load a valid block (results are not stored).
  const int nbl[2] = {min(nbw0, NBT - 1), min(nbw0 + 1, NBT - 1)};

  // The A tile goes global -> LDS by DMA (global_load_lds_dwordx4): lane l of
  // wave w's chunk i writes the 16-byte slot p = (NW*i + w)*64 + l, which holds
  // (row p/8, k-chunk (p%8) ^ ((row/2)%8)) of the swizzled tile. Rows past M
  // load row M-1 (their results are not stored). Byte offsets fit 32 bits:
  // the host checks M*K.
  uint32_t doff[ACH];
#pragma unroll
  for (int i = 0; i < ACH; i++) {
    const int p = (NW * i + wave) * 64 + lane, row = p >> 3, kc = (p & 7) ^ ((row >> 1) & 7);
    doff[i] = ((uint32_t)min(m0 + row, g.M - 1) * (uint32_t)g.K + (uint32_t)(kc * 8)) * 2u;
  }
  const char* xa = (const char*)g.x;
  const char* xl = (const char*)g.xlo;  // EX: the lo plane (same offsets)
  PipeB<FORM> bq[4][2];  // B(k) in slot k % 4, all four live
  // A wave's scales (lanes 0-15: blocks nbl[0], nbl[1]) and zeros (lanes
  // 16-31) of one k-step are 128-byte runs of the packed arrays.
  const int szl = lane & 15, szb = szl >> 3;
  const char* szsrc = (const char*)((lane >> 4) ? g.wz : g.ws) +
                      ((size_t)nbl[szb] * KS * 64 + (size_t)(szl & 7) * 8) * 2;
  const bool szlane = LS && (lane < (FORM == TGOHIP_FORM_I4_TGO ? 32 : 16));
#define PIPE_DMA_A(ks, stage)                                                          \
  do {                                                                                 \
    _Pragma("unroll") for (int i = 0; i < ACH; i++)                                    \
        __builtin_amdgcn_global_load_lds(                                              \
            (const __attribute__((address_space(1))) void*)(xa + (size_t)(ks) * 128 + doff[i]), \
            (__attribute__((address_space(3))) void*)(As[stage] + aq + (NW * i + wave) * 512), 16, 0, 0); \
    if (EX)                                                                            \
      _Pragma("unroll") for (int i = 0; i < ACH; i++)                                  \
          __builtin_amdgcn_global_load_lds(                                            \
              (const __attribute__((address_space(1))) void*)(xl + (size_t)(ks) * 128 + doff[i]), \
              (__attribute__((address_space(3))) void*)(As[stage] + aq + MW * 64 + (NW * i + wave) * 512), \
              16, 0, 0);                                                               \
    if (LS && szlane)                                                                  \
      __builtin_amdgcn_global_load_lds(                                                \
          (const __attribute__((address_space(1))) void*)(szsrc + (size_t)(ks) * 128), \
          (__attribute__((address_space(3))) void*)(Sz[stage] + sq + wave * 256), 16, 0, 0); \
  } while (0)

  float16_t acc[MB][2];
#pragma unroll
  for (int mb = 0; mb < MB; mb++)
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mb][b][r] = 0.f;
  float16_t accg[FX ? MB : 1][2];  // FX: the current scale group's inner sums
  const float16_t zero16 = {};

  // A(k) (and the scales of B(k) when they travel by LDS) sits in LDS stage
  // k % 4, DMA'd in the middle of step k-3; B(k) in register slot k % 4,
  // loaded at the start of step k-3 (the slot of B(k-4), whose last read
  // was in step k-4; three steps ahead cut the M = 128 gate/up from 46 to
  // 41 us). Each step reads the next step's first
  // fragments during its last substep, so the MFMAs run on across step
  // boundaries. One barrier per step, in its middle. Before it a wave waits
  // for its own DMA of stage k+1 (issued at step k-2: the vector memory
  // operations issued since are B(k+2), stage k+2's DMA and B(k+3)) and for its
  // LDS reads; past it, stage k+1 is visible to every wave, and every wave is
  // done reading stage k-1, which the DMA of stage k+3 issued right after the
  // barrier reuses. The barrier carries no memory fence: a fence would wait
  // for every DMA in flight.
  auto kpos = [&](int k) { return ks0 + min(k, nk - 1); };
  // Substep fragments: A rows (hi; with EX also lo) and B blocks (hi; with EX
  // the exact weight's lo part too).
  half8_t afc[MB], bfc[2], afcl[MB], bfcl[2];
  constexpr int LOP = MW * 8;  // half8s from a stage's hi plane to its lo plane
  auto read_a = [&](const half8_t* A, int kc, half8_t (&ah)[MB], half8_t (&al)[MB]) {
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
      ah[mb] = A[a_slot(mb * 32 + c32, kc)];
      if (EX) al[mb] = A[LOP + a_slot(mb * 32 + c32, kc)];
    }
  };
  auto read_b = [&](const PipeB<FORM>(&bb)[2], int j, const half_t* sz, half8_t (&bh)[2],
                    half8_t (&bl)[2]) {
#pragma unroll
    for (int b = 0; b < 2; b++) {
      if constexpr (FX) bh[b] = i4_sym_codes(word_of(bb[b].p, j));
      else if constexpr (EX) pipe_bfrag_x(bb[b], j, sz, b, h, bh[b], bl[b]);
      else bh[b] = pipe_bfrag(bb[b], j, sz, b, h);
    }
  };
  if (nk > 0) {  // nk is then a multiple of 4 (the host guarantees it)
#pragma unroll
    for (int b = 0; b < 2; b++) load_pipeb(g, nbl[b], kpos(0), lane, bq[0][b]);
#pragma unroll
    for (int b = 0; b < 2; b++) load_pipeb(g, nbl[b], kpos(1), lane, bq[1][b]);
#pragma unroll
    for (int b = 0; b < 2; b++) load_pipeb(g, nbl[b], kpos(2), lane, bq[2][b]);
    PIPE_DMA_A(kpos(0), 0);
    PIPE_DMA_A(kpos(1), 1);
    PIPE_DMA_A(kpos(2), 2);
    __builtin_amdgcn_s_waitcnt(0);  // all counters: the prologue's loads and DMA
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read_a((const half8_t*)(As[0] + aq), h, afc, afcl);
    read_b(bq[0], 0, Sz[0] + sq + wave * 256, bfc, bfcl);
  }
  for (int kk = 0; kk < nk; kk += 4) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
#pragma unroll
      for (int b = 0; b < 2; b++) load_pipeb(g, nbl[b], kpos(kk + u + 3), lane, bq[(u + 3) % 4][b]);
      // Keep the loads issued here, ahead of the MFMAs: the scheduler would
      // otherwise sink them next to their use and expose their latency.
      __builtin_amdgcn_sched_barrier(0);
      // Raised wave priority through the MFMA phase: of the two waves sharing
      // a SIMD, the one issuing MFMAs goes first.
      __builtin_amdgcn_s_setprio(1);
      const half8_t* A = (const half8_t*)(As[u] + aq);
      const half8_t* An = (const half8_t*)(As[(u + 1) % 4] + aq);
      // Substep j's MFMAs run while the next substep's A fragments are read
      // from LDS and its B fragments dequantized; the group barriers
      // interleave them (1 MFMA, 1 LDS read, 5 VALU) so the matrix core stays
      // fed.
#pragma unroll
      for (int j = 0; j < 4; j++) {
        half8_t afn[MB], bfn[2], afnl[MB], bfnl[2];
        if (j < 3) {
          read_a(A, 2 * (j + 1) + h, afn, afnl);
          read_b(bq[u], j + 1, Sz[u] + sq + wave * 256, bfn, bfnl);
        } else {
          read_a(An, h, afn, afnl);
          read_b(bq[(u + 1) % 4], 0, Sz[(u + 1) % 4] + sq + wave * 256, bfn, bfnl);
        }
        if constexpr (FX) {
          // substeps 0-1 are the k-step's first scale group, 2-3 its second;
          // an even substep starts the group's sums, an odd one ends them
          // and scales them into acc
#pragma unroll
          for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int b = 0; b < 2; b++)
              accg[mb][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                  afc[mb], bfc[b], (j & 1) ? accg[mb][b] : zero16, 0, 0, 0);
#pragma unroll
          for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int b = 0; b < 2; b++)
              accg[mb][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afcl[mb], bfc[b], accg[mb][b], 0, 0, 0);
          if (j & 1) {
            // The scaling reads the group's last MFMAs, so this wave has no
            // MFMA to issue beside it: at the lower priority the other wave
            // on the SIMD issues first (the C4 step 40.1-40.5 -> 39.1 ms;
            // gate/up 407 -> 390-399 us, QKV 116 -> 106-111 us). With two k
            // groups per workgroup the isolated block spilled more (18
            // VGPRs, not 8-11), so they keep the interleave below. The
            // lane's column scale of this group: bq[u] holds step u's two
            // per lane column.
            if constexpr (KQ == 1) {
              __builtin_amdgcn_sched_barrier(0);
              __builtin_amdgcn_s_setprio(0);
            }
#pragma unroll
            for (int b = 0; b < 2; b++) {
              union { uint32_t u; half2_t h; } sc;
              sc.u = bq[u][b].s;
              const float s = (float)sc.h[j >> 1];
#pragma unroll
              for (int mb = 0; mb < MB; mb++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[mb][b][r] = __builtin_fmaf(accg[mb][b][r], s, acc[mb][b][r]);
            }
            if constexpr (KQ == 1) {
              __builtin_amdgcn_s_setprio(1);
              __builtin_amdgcn_sched_barrier(0);
            }
          }
        } else {
#pragma unroll
          for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int b = 0; b < 2; b++)
              acc[mb][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afc[mb], bfc[b], acc[mb][b], 0, 0, 0);
        }
        if constexpr (EX && !FX) {
          // the two correction products, each pass over every block, so no
          // MFMA waits on the one just issued into the same accumulator
#pragma unroll
          for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int b = 0; b < 2; b++)
              acc[mb][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afcl[mb], bfc[b], acc[mb][b], 0, 0, 0);
#pragma unroll
          for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int b = 0; b < 2; b++)
              acc[mb][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afc[mb], bfcl[b], acc[mb][b], 0, 0, 0);
        }
        if constexpr (FX) {
          // 8 MFMAs (64-row tiles), 4 LDS reads, the codes' 18 VALU; with
          // two k groups an odd substep's 64 scaling fmas fill its VALU
          // slots (with one, its MFMA region is scheduled freely, above)
          if ((j & 1) == 0)
#pragma unroll
            for (int q = 0; q < 4; q++) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
              __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
              __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
              __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
            }
          else if (KQ == 2)
#pragma unroll
            for (int q = 0; q < 4; q++) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
              __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read
              __builtin_amdgcn_sched_group_barrier(0x002, 10, 0);  // VALU
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
              __builtin_amdgcn_sched_group_barrier(0x002, 10, 0);  // VALU
            }
        } else if constexpr (EX) {
          // 12 MFMAs (64-row tiles), 4 LDS reads, the B pairs' 36 VALU
#pragma unroll
          for (int q = 0; q < 4; q++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          }
        } else {
#pragma unroll
          for (int q = 0; q < 4; q++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // VALU
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // VALU
          }
        }
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
          afc[mb] = afn[mb];
          afcl[mb] = afnl[mb];
        }
#pragma unroll
        for (int b = 0; b < 2; b++) {
          bfc[b] = bfn[b];
          bfcl[b] = bfnl[b];
        }
        if (j == 1) {
          __builtin_amdgcn_sched_barrier(0);
          // vmcnt(2 * B loads + A DMA + scale DMA), expcnt untouched, lgkmcnt(0);
          // vmcnt's low 4 bits sit at 3:0 and its high 2 at 15:14
          constexpr int VMC = 2 * pipe_b_loads<FORM>() + AP * ACH + (LS ? 1 : 0);
          static_assert(VMC < 64, "vmcnt fits 6 bits");
          __builtin_amdgcn_s_waitcnt((VMC & 15) | ((VMC >> 4) << 14) | (7 << 4));
          asm volatile("" ::: "memory");
          __builtin_amdgcn_s_barrier();
          asm volatile("" ::: "memory");
          PIPE_DMA_A(kpos(kk + u + 3), (u + 3) % 4);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // no DMA into LDS outlives the loop
  if constexpr (KQ == 2) {
    // Group 1's sums to group 0 through the A ring (stage w of column wave
    // w: MW * 256 bytes, lane-contiguous float4s), added in that order.
    __syncthreads();
    float4_t* red = (float4_t*)(wave == 0 ? As0 : wave == 1 ? As1 : wave == 2 ? As2 : As3);
    if (kq == 1) {
#pragma unroll
      for (int mb = 0; mb < MB; mb++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
          for (int r4 = 0; r4 < 4; r4++)
            red[((mb * 2 + b) * 4 + r4) * 64 + lane] =
                float4_t{acc[mb][b][4 * r4], acc[mb][b][4 * r4 + 1], acc[mb][b][4 * r4 + 2],
                         acc[mb][b][4 * r4 + 3]};
    }
    __syncthreads();
    if (kq == 1) return;
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
      for (int b = 0; b < 2; b++)
#pragma unroll
        for (int r4 = 0; r4 < 4; r4++) {
          const float4_t o = red[((mb * 2 + b) * 4 + r4) * 64 + lane];
#pragma unroll
          for (int e = 0; e < 4; e++) acc[mb][b][4 * r4 + e] += o[e];
        }
  }
  if constexpr (EPI == EPI_QKROPE) {
    // The tile (64 rows x two 128-wide heads; the host launches this only
    // unsplit, with one k group, 64-row tiles and whole heads per tile) goes
    // through LDS, rows 16i..16i+15 in stage i of the A ring, so that each
    // half wave can take a head row with four consecutive dims per lane, as
    // qk_rope_kv_kernel does; the angles come from the step's rope table.
    static_assert(MW == 64 && NW == 4 && KQ == 1, "one 64 x 256 f32 tile fills the A ring");
    __syncthreads();  // every wave's last ring reads are done (its DMAs waited above)
    // (a stage picked by value: an array of the stages' addresses would need
    // a static initializer)
    auto ring = [](int i, half_t* s0, half_t* s1, half_t* s2, half_t* s3) {
      return (float*)(i == 0 ? s0 : i == 1 ? s1 : i == 2 ? s2 : s3);
    };
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
      for (int b = 0; b < 2; b++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int row = mb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          ring(row >> 4, As0, As1, As2, As3)[(row & 15) * 256 + wave * 64 + b * 32 + c32] = acc[mb][b][r];
        }
    __syncthreads();
    // wave w takes rows w, w + 4, ...; its half waves the tile's two heads
    for (int row = wave; row < MW; row += NW) {
      const int t = m0 + row;
      if (t >= g.M) break;  // wave-uniform
      const float4_t v =
          *(const float4_t*)(ring(row >> 4, As0, As1, As2, As3) + (row & 15) * 256 + h * 128 + 4 * c32);
      const float4_t cs = qa.rope[(size_t)t * 32 + c32];
      qk_head_row(qa, t, 2 * tn + h, c32, v, qa.slots[t],
                  [&](bool, int, float& c0, float& s0, float& c1, float& s1) {
                    c0 = cs[0];
                    s0 = cs[1];
                    c1 = cs[2];
                    s1 = cs[3];
                  });
    }
  } else {
    gemm_epilogue<EPI, MB>(g, acc, m0, nbw0, nbv, h, c32, nsplit > 1, split);
  }
#undef PIPE_DMA_A
}

// a += p[0], p[plane], ... p[(N-1) plane] in that order, every load issued
// before the first add.
template <int N>
__device__ __forceinline__ void add_split_values(float& a, const float* p, size_t plane) {
  float v[N];
#pragma unroll
  for (int u = 0; u < N; u++) v[u] = p[(size_t)u * plane];
#pragma unroll
  for (int u = 0; u < N; u++) a += v[u];
}
// Sum of the split partials at p (planes `plane` apart), in split order, up
// to eight loads in flight at a time.
__device__ __forceinline__ float sum_split_values(const float* p, int splits, size_t plane) {
  float a = 0.f;
  for (int s0 = 0; s0 < splits; s0 += 8) {
    const float* q = p + (size_t)s0 * plane;
    switch (min(splits - s0, 8)) {
      case 1: add_split_values<1>(a, q, plane); break;
      case 2: add_split_values<2>(a, q, plane); break;
      case 3: add_split_values<3>(a, q, plane); break;
      case 4: add_split_values<4>(a, q, plane); break;
      case 5: add_split_values<5>(a, q, plane); break;
      case 6: add_split_values<6>(a, q, plane); break;
      case 7: add_split_values<7>(a, q, plane); break;
      default: add_split_values<8>(a, q, plane); break;
    }
  }
  return a;
}

// Sums split-K partials in split order and applies the epilogue.
template <int EPI>
__global__ void gemm_reduce_kernel(GemmArgs g, int splits) {
  constexpr bool SW = EPI == EPI_SWIGLU_F16 || EPI == EPI_SWIGLU_F32 || EPI == EPI_SWIGLU_X2;
  const int outN = SW ? g.N / 2 : g.N;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)g.M * outN) return;
  const int row = (int)(i / outN), col = (int)(i % outN);
  const size_t plane = g.pstride;
  if (SW) {
    const int gc = (col / 32) * 64 + (col % 32), uc = gc + 32;
    const float ga = sum_split_values(g.part + (size_t)row * g.N + gc, splits, plane);
    const float ua = sum_split_values(g.part + (size_t)row * g.N + uc, splits, plane);
    store_swiglu<EPI>(g, i, silu_f(ga) * ua);
  } else {
    const float a = sum_split_values(g.part + i, splits, plane);
    if (EPI == EPI_F32) ((float*)g.y)[i] = a;
    else if (EPI == EPI_F16) ((half_t*)g.y)[i] = (half_t)a;
    else ((float*)g.y)[i] += a;
  }
}

// gemm_reduce_kernel with four consecutive outputs per thread (the host uses
// it when the output row is a multiple of 4 wide; a SwiGLU's four then stay
// in one 32-column block): float4 loads from every split's plane, up to
// eight splits' loads in flight, each element summed in split order from 0
// as sum_split_values sums it, so the results are the same to the bit.
template <int EPI>
__global__ void gemm_reduce4_kernel(GemmArgs g, int splits) {
  constexpr bool SW = EPI == EPI_SWIGLU_F16 || EPI == EPI_SWIGLU_F32 || EPI == EPI_SWIGLU_X2;
  const int outN = SW ? g.N / 2 : g.N;
  const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= (size_t)g.M * outN) return;
  const int row = (int)(i / outN), col = (int)(i % outN);
  auto sum4 = [&](size_t off) {
    float4_t a = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < splits; s0 += 8) {
      const int n = min(splits - s0, 8);
      float4_t v[8];
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (u < n) v[u] = *(const float4_t*)(g.part + (size_t)(s0 + u) * g.pstride + off);
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (u < n) {
#pragma unroll
          for (int e = 0; e < 4; e++) a[e] += v[u][e];
        }
    }
    return a;
  };
  if (SW) {
    const size_t gc = (size_t)row * g.N + (col / 32) * 64 + (col % 32);
    const float4_t ga = sum4(gc), ua = sum4(gc + 32);
    float4_t v;
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = silu_f(ga[e]) * ua[e];
    if (EPI == EPI_SWIGLU_F32) {
      *(float4_t*)((float*)g.y + i) = v;
    } else {
      const half4_t hv = {(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
      *(half4_t*)((half_t*)g.y + i) = hv;
      if (EPI == EPI_SWIGLU_X2) {
        half4_t lv;
#pragma unroll
        for (int e = 0; e < 4; e++) lv[e] = (half_t)(v[e] - (float)hv[e]);
        *(half4_t*)((half_t*)g.y + (size_t)g.M * outN + i) = lv;
      }
    }
  } else {
    const float4_t a = sum4(i);
    if (EPI == EPI_F32) {
      *(float4_t*)((float*)g.y + i) = a;
    } else if (EPI == EPI_F16) {
      *(half4_t*)((half_t*)g.y + i) = half4_t{(half_t)a[0], (half_t)a[1], (half_t)a[2], (half_t)a[3]};
    } else {
      float4_t y = *(const float4_t*)((float*)g.y + i);
#pragma unroll
      for (int e = 0; e < 4; e++) y[e] += a[e];
      *(float4_t*)((float*)g.y + i) = y;
    }
  }
}

// ---------------------------------------------------------------------------
// repack: canonical host forms (already on the device) -> fragment-major
// ---------------------------------------------------------------------------
struct RepackArgs {
  const void* plane;
  const uint16_t* scales;
  const uint16_t* zeros;
  void* wp;
  uint16_t* ws;
  uint16_t* wz;
  int K, N;            // the sub-weight's shape
  int nb_stride, nb_off;  // its n-block nb lands at nb*nb_stride + nb_off
};

__device__ __forceinline__ int nib_slot(int e) { return (e & 1) * 4 + (e >> 1); }
__device__ __forceinline__ int byte_slot(int e) { return (e & 1) * 2 + (e >> 1); }  // 0,2,1,3

// One thread per (nb, ks, lane).
template <int FORM>
__global__ void repack_kernel(RepackArgs a) {
  const int KS = a.K / 64, NBT = a.N / 32;
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (size_t)NBT * KS * 64) return;
  const int lane = (int)(t % 64), ks = (int)((t / 64) % KS), nb = (int)(t / 64 / KS);
  const int h = lane >> 5, n = nb * 32 + (lane & 31);
  const size_t N = (size_t)a.N;
  const int onb = nb * a.nb_stride + a.nb_off;
  const size_t ot = ((size_t)onb * KS + ks) * 64 + lane;  // output slot
  for (int j = 0; j < 4; j++) {
    const int kb = ks * 64 + 16 * j + 8 * h;
    if (FORM == TGOHIP_FORM_F16) {
      uint16_t* dst = (uint16_t*)a.wp + ot * 32 + j * 8;
      for (int e = 0; e < 8; e++) dst[e] = ((const uint16_t*)a.plane)[(size_t)(kb + e) * N + n];
    } else if (FORM == TGOHIP_FORM_I4_SYM) {
      uint32_t w = 0;
      for (int e = 0; e < 8; e++) {
        const int k = kb + e;
        const uint32_t word = ((const uint32_t*)a.plane)[(size_t)(k / 8) * N + n];
        w |= ((word >> (4 * (k % 8))) & 15u) << (4 * nib_slot(e));
      }
      ((uint32_t*)a.wp)[ot * 4 + j] = w;
    } else if (FORM == TGOHIP_FORM_I4_TGO) {
      uint32_t w = 0;
      for (int e = 0; e < 8; e++) {
        const size_t i = (size_t)(kb + e) * N + n;
        const uint32_t q = (((const uint32_t*)a.plane)[i / 8] >> (4 * (i % 8))) & 15u;
        w |= q << (4 * nib_slot(e));
      }
      ((uint32_t*)a.wp)[ot * 4 + j] = w;
    } else {
      uint32_t w[2] = {0, 0};
      for (int e = 0; e < 8; e++) {
        const size_t i = (size_t)(kb + e) * N + n;
        const uint32_t b = (uint32_t)((int)((const int8_t*)a.plane)[i] + 128) & 255u;
        w[e >> 2] |= b << (8 * byte_slot(e & 3));
      }
      ((uint32_t*)a.wp)[ot * 8 + j * 2] = w[0];
      ((uint32_t*)a.wp)[ot * 8 + j * 2 + 1] = w[1];
    }
    // per-k scales (and zeros) for I8 / I4_TGO: written by lanes 0 and 32.
    if ((FORM == TGOHIP_FORM_I8 || FORM == TGOHIP_FORM_I4_TGO) && (lane & 31) == 0) {
      const size_t o = ((((size_t)onb * KS + ks) * 4 + j) * 2 + h) * 8;
      for (int e = 0; e < 8; e++) {
        const size_t i = (size_t)(kb + e) * N + n;  // n is the block's first column
        if (FORM == TGOHIP_FORM_I8) {
          a.ws[o + e] = a.scales[i / 32];
        } else {
          a.ws[o + e] = a.scales[i / 128];
          // 1024 + z, exact in f16 for an integer zero in [0, 1023]
          const float z = (float)(*(const half_t*)&a.zeros[i / 128]);
          const half_t zz = (half_t)(1024.f + z);
          a.wz[o + e] = *(const uint16_t*)&zz;
        }
      }
    }
  }
  if (FORM == TGOHIP_FORM_I4_SYM && h == 0) {
    const size_t o = (((size_t)onb * KS + ks) * 32 + (lane & 31)) * 2;
    a.ws[o] = a.scales[(size_t)(2 * ks) * N + n];
    a.ws[o + 1] = a.scales[(size_t)(2 * ks + 1) * N + n];
  }
}

// Dequantizes a packed weight to [K,N]: f32 exactly ((q - z) * s in f32) or the
// f16 the MFMA path multiplies (the same device functions as the GEMM).
template <int FORM, bool F16OUT>
__global__ void dequant_kernel(GemmArgs g, void* out) {
  const int KS = g.K / 64, NBT = g.N / 32;
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (size_t)NBT * KS * 64) return;
  const int lane = (int)(t % 64), ks = (int)((t / 64) % KS), nb = (int)(t / 64 / KS);
  const int h = lane >> 5, n = nb * 32 + (lane & 31);
  BRaw<FORM> r;
  load_braw(g, nb, ks, lane, r);
  for (int j = 0; j < 4; j++) {
    const int kb = ks * 64 + 16 * j + 8 * h;
    if (F16OUT) {
      const half8_t f = bfrag(r, j);
      for (int e = 0; e < 8; e++) ((half_t*)out)[(size_t)(kb + e) * g.N + n] = f[e];
    } else {
      for (int e = 0; e < 8; e++) {
        float v;
        if constexpr (FORM == TGOHIP_FORM_F16) {
          U16B c;
          c.u = r.p[j];
          v = (float)c.h[e];
        } else if constexpr (FORM == TGOHIP_FORM_I4_SYM) {
          const uint32_t q = (word_of(r.p, j) >> (4 * nib_slot(e))) & 15u;
          union { uint32_t u; half2_t hh; } sc;
          sc.u = r.s;
          v = (float)((int)q - 8) * (float)(j < 2 ? sc.hh[0] : sc.hh[1]);
        } else if constexpr (FORM == TGOHIP_FORM_I4_TGO) {
          const uint32_t q = (word_of(r.p, j) >> (4 * nib_slot(e))) & 15u;
          U16B sv, zv;
          sv.u = r.s[j];
          zv.u = r.z[j];
          v = ((float)q - ((float)zv.h[e] - 1024.f)) * (float)sv.h[e];
        } else {
          const uint4 qq = r.p[j >> 1];
          const uint32_t w = (e < 4) ? ((j & 1) ? qq.z : qq.x) : ((j & 1) ? qq.w : qq.y);
          const uint32_t bb = (w >> (8 * byte_slot(e & 3))) & 255u;
          U16B sv;
          sv.u = r.s[j];
          v = (float)((int)bb - 128) * (float)sv.h[e];
        }
        ((float*)out)[(size_t)(kb + e) * g.N + n] = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

size_t packed_payload_bytes(int form, int K, int N) {
  const size_t slots = (size_t)(N / 32) * (K / 64) * 64;
  switch (form) {
    case TGOHIP_FORM_F16: return slots * 64;
    case TGOHIP_FORM_I8: return slots * 32;
    default: return slots * 16;
  }
}
size_t packed_scale_halves(int form, int K, int N) {
  switch (form) {
    case TGOHIP_FORM_I4_SYM: return (size_t)(N / 32) * (K / 64) * 32 * 2;
    case TGOHIP_FORM_I8:
    case TGOHIP_FORM_I4_TGO: return (size_t)(N / 32) * (K / 64) * 4 * 2 * 8;
    default: return 0;
  }
}

int repack_enqueue(int form, const void* plane, const uint16_t* scales, const uint16_t* zeros,
                   int K, int N, PackedWeight& w, int nb_stride, int nb_off, hipStream_t st) {
  RepackArgs a{plane, scales, zeros, w.wp, (uint16_t*)w.ws, (uint16_t*)w.wz, K, N, nb_stride, nb_off};
  const size_t threads = (size_t)(N / 32) * (K / 64) * 64;
  const dim3 grid((unsigned)((threads + 255) / 256)), blk(256);
  switch (form) {
    case TGOHIP_FORM_F16: hipLaunchKernelGGL(repack_kernel<TGOHIP_FORM_F16>, grid, blk, 0, st, a); break;
    case TGOHIP_FORM_I8: hipLaunchKernelGGL(repack_kernel<TGOHIP_FORM_I8>, grid, blk, 0, st, a); break;
    case TGOHIP_FORM_I4_TGO: hipLaunchKernelGGL(repack_kernel<TGOHIP_FORM_I4_TGO>, grid, blk, 0, st, a); break;
    case TGOHIP_FORM_I4_SYM: hipLaunchKernelGGL(repack_kernel<TGOHIP_FORM_I4_SYM>, grid, blk, 0, st, a); break;
  }
  TGOHIP_HIP(hipGetLastError());
  return 0;
}

int dequant_enqueue(const PackedWeight& w, void* out, bool f16out, hipStream_t st) {
  GemmArgs g{};
  g.wp = w.wp;
  g.ws = w.ws;
  g.wz = w.wz;
  g.K = w.K;
  g.N = w.N;
  const size_t threads = (size_t)(w.N / 32) * (w.K / 64) * 64;
  const dim3 grid((unsigned)((threads + 255) / 256)), blk(256);
#define DQ(F)                                                                              \
  if (f16out) hipLaunchKernelGGL((dequant_kernel<F, true>), grid, blk, 0, st, g, out);     \
  else hipLaunchKernelGGL((dequant_kernel<F, false>), grid, blk, 0, st, g, out);
  switch (w.form) {
    case TGOHIP_FORM_F16: DQ(TGOHIP_FORM_F16); break;
    case TGOHIP_FORM_I8: DQ(TGOHIP_FORM_I8); break;
    case TGOHIP_FORM_I4_TGO: DQ(TGOHIP_FORM_I4_TGO); break;
    case TGOHIP_FORM_I4_SYM: DQ(TGOHIP_FORM_I4_SYM); break;
  }
#undef DQ
  TGOHIP_HIP(hipGetLastError());
  return 0;
}

// ---- small M: the weight stream is the cost ---------------------------------
// At most 32 activation rows. A workgroup owns CB 32-column blocks (two for
// the SwiGLU epilogue, which pairs gate and up blocks) over all of K; its W
// waves each stream one contiguous share of the k-steps (K/64/W of them) as
// a run of 1 KiB (int4) weight bursts with gemv_depth<FORM>() k-steps of
// loads in flight, computing on the oldest while the rest arrive. The waves'
// sums meet in LDS and are added in wave order, so the result is
// deterministic and one launch does the whole product.
//   Staged (1-8 rows, M*(K+8)*2 <= kGemvStageBytes): the activation rows are
//     copied into LDS once per workgroup (after the first weight loads are
//     issued; rows K + 8 halves apart, so the rows a read takes sit in
//     different banks) and the MFMA A operand is read from there, so the weight stream
//     is the only vector-memory traffic in the loop (measured at M = 1: LM
//     head 88 -> 65 us, gate/up 17 -> 14 us against A loads from global
//     memory). The product is v_mfma_f32_16x16x32_f16, half the matrix work
//     per weight of 32x32x16: its hardware k slot (kq = lane/16, e) meets the
//     weight lane whose fragment holds column n + 16 (kq % 2), k offset
//     8 (kq / 2) + e of the substep, so an A operand that carries row i of k
//     half kq/2 in A row i when kq is even and in A row 8 + i when kq is odd
//     (zero otherwise) puts columns 0-15 of the block in D rows 0-7 and
//     columns 16-31 in D rows 8-15.
//   Direct (9-32 rows, or a K too long to stage): v_mfma_f32_32x32x16_f16 on
//     the fragment as laid out, the A operand loaded from global memory with
//     the weights (small and L2-resident; rows >= M are zero).
template <int FORM> constexpr int gemv_depth() {
  return FORM == TGOHIP_FORM_I8 || FORM == TGOHIP_FORM_I4_TGO ? 2 : 4;
}
// Waves per workgroup the registers allow (128 VGPRs at 16 waves): 16 for
// one column block of the int4-sym and int8 packs, 8 otherwise.
constexpr int gemv_max_waves(int form, int cb) {
  return cb == 1 && (form == TGOHIP_FORM_I4_SYM || form == TGOHIP_FORM_I8) ? 16 : 8;
}
constexpr int kGemvStageBytes = (64 << 10) + 128;  // 8 rows of K = 4096, padded
__host__ __device__ constexpr int gemv_stage_stride(int K) { return K + 8; }

template <int EPI, int CB>
__device__ __forceinline__ void gemv_store(const GemmArgs& g, int nbw0, const bool (&nbv)[CB], int row,
                                           int col, const float (&v)[CB]) {
  if constexpr (EPI == EPI_SWIGLU_F16 || EPI == EPI_SWIGLU_F32 || EPI == EPI_SWIGLU_X2) {
    if (!nbv[CB - 1]) return;
    const size_t off = (size_t)row * (g.N / 2) + (nbw0 >> 1) * 32 + col;
    store_swiglu<EPI>(g, off, silu_f(v[0]) * v[CB - 1]);
  } else {
#pragma unroll
    for (int b = 0; b < CB; b++) {
      if (!nbv[b]) continue;
      const size_t off = (size_t)row * g.N + (nbw0 + b) * 32 + col;
      if (EPI == EPI_F32) ((float*)g.y)[off] = v[b];
      else if (EPI == EPI_F16) ((half_t*)g.y)[off] = (half_t)v[b];
      else ((float*)g.y)[off] += v[b];
    }
  }
}

// STAGED: the staged 1-8 row form (dynamic LDS of M*K halves); else direct.
template <int FORM, int EPI, int CB, int W, bool STAGED>
__global__ __launch_bounds__(64 * W) void gemm_gemv_kernel(GemmArgs g) {
  constexpr int D = gemv_depth<FORM>();
  constexpr int ROWS = STAGED ? 8 : 32;
  constexpr int OUT = CB * ROWS * 32;  // a wave's sums: CB blocks of ROWS rows x 32 columns
  __shared__ float red[W][OUT];
  extern __shared__ __attribute__((aligned(16))) half_t xs[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int NBT = g.N / 32;
  const int nbw0 = blockIdx.x * CB;
  bool nbv[CB];
  int nbl[CB];
#pragma unroll
  for (int b = 0; b < CB; b++) {
    nbv[b] = nbw0 + b < NBT;
    nbl[b] = min(nbw0 + b, NBT - 1);
  }
  const int kw = (g.K / 64) / W, ks0 = wave * kw;  // kw % D == 0
  // The lane's activation row and k half, and whether it carries one.
  int arow, ah;
  bool av;
  if constexpr (STAGED) {
    const int ai = lane & 15, kq = lane >> 4;
    arow = ai & 7;
    ah = kq >> 1;
    av = ((ai < 8) == ((kq & 1) == 0)) && arow < g.M;
  } else {
    arow = lane & 31;
    ah = lane >> 5;
    av = arow < g.M;
  }
  const half_t* xr = (STAGED ? (const half_t*)xs : (const half_t*)g.x) +
                     (size_t)(av ? arow : 0) * (STAGED ? gemv_stage_stride(g.K) : g.K) + 8 * ah;

  typedef typename std::conditional<STAGED, float4_t, float16_t>::type Acc;
  Acc acc[CB];
#pragma unroll
  for (int b = 0; b < CB; b++)
#pragma unroll
    for (int r = 0; r < (STAGED ? 4 : 16); r++) acc[b][r] = 0.f;
  BRaw<FORM> bq[D][CB];
  half8_t aq[D][4];
  // A operand of k-step ks: from LDS (staged) or global memory, zero where the
  // lane carries no row.
  auto load_a = [&](half8_t(&a)[4], int ks) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      if constexpr (STAGED) {
        half8_t v = {0, 0, 0, 0, 0, 0, 0, 0};
        if (av) v = *(const half8_t*)(xr + ks * 64 + 16 * j);
        a[j] = v;
      } else {
        const half8_t v = *(const half8_t*)(xr + ks * 64 + 16 * j);
        a[j] = av ? v : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
  };
  auto load = [&](int d, int ks) {
#pragma unroll
    for (int b = 0; b < CB; b++) load_braw<true>(g, nbl[b], ks, lane, bq[d][b]);
    if constexpr (!STAGED) load_a(aq[d], ks);
  };
#pragma unroll
  for (int d = 0; d < D; d++) load(d, ks0 + d);
  if constexpr (STAGED) {
    // Every 16-byte chunk's load is issued before the first is written, so
    // the copy costs one L2 round trip.
    constexpr int SC = (kGemvStageBytes / 16 + 64 * W - 1) / (64 * W);
    const half_t* x = (const half_t*)g.x;
    const int nch = g.M * g.K / 8;
    half8_t t[SC];
#pragma unroll
    for (int u = 0; u < SC; u++)
      if (tid + u * 64 * W < nch) t[u] = *(const half8_t*)(x + 8 * (tid + u * 64 * W));
#pragma unroll
    for (int u = 0; u < SC; u++) {
      const int i = 8 * (tid + u * 64 * W);
      if (i < 8 * nch) {
        const int row = i / g.K;
        *(half8_t*)(xs + row * gemv_stage_stride(g.K) + (i - row * g.K)) = t[u];
      }
    }
    __syncthreads();
  }
  for (int i = 0; i < kw; i += D) {
#pragma unroll
    for (int d = 0; d < D; d++) {
      if constexpr (STAGED) load_a(aq[d], ks0 + i + d);
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int b = 0; b < CB; b++) {
          if constexpr (STAGED)
            acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq[d][j], bfrag(bq[d][b], j), acc[b], 0, 0, 0);
          else
            acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(aq[d][j], bfrag(bq[d][b], j), acc[b], 0, 0, 0);
        }
      if (i + d + D < kw) load(d, ks0 + i + d + D);
    }
  }
  if constexpr (STAGED) {
    // Lane l holds D[4(l/16) + r][l%16]: row 4((l/16)%2) + r of column l%16 + 16(l/32).
    const int row0 = 4 * ((lane >> 4) & 1), col = (lane & 15) + 16 * (lane >> 5);
#pragma unroll
    for (int b = 0; b < CB; b++)
#pragma unroll
      for (int r = 0; r < 4; r++)
        if (row0 + r < g.M) red[wave][b * 256 + (row0 + r) * 32 + col] = acc[b][r];
  } else {
    // Lane (c32, h) holds D[8(r/4) + 4h + r%4][c32] of each block.
    const int h = lane >> 5, c32 = lane & 31;
#pragma unroll
    for (int b = 0; b < CB; b++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = 8 * (r >> 2) + 4 * h + (r & 3);
        if (row < g.M) red[wave][b * 1024 + row * 32 + c32] = acc[b][r];
      }
  }
  __syncthreads();
  for (int rc = tid; rc < g.M * 32; rc += 64 * W) {
    float v[CB];
#pragma unroll
    for (int b = 0; b < CB; b++) {
      v[b] = 0.f;
#pragma unroll
      for (int w = 0; w < W; w++) v[b] += red[w][b * ROWS * 32 + rc];
    }
    gemv_store<EPI, CB>(g, nbw0, nbv, rc >> 5, rc & 31, v);
  }
}

// Launch shape of the small-M kernels: CB column blocks (2 for SwiGLU), the
// form (staged or direct) and W waves per workgroup: the fewest of the
// candidates (8, 16 staged; 4, 8, 16 direct) that put about three waves on
// every SIMD (12 per CU), within the form's cap and with each wave's share of
// K a whole multiple of the load depth; w = 0 when none fits. Measured at
// M = 1: the staged LM head runs best at 8 waves (65 us; 66 at 4, 68 at 16),
// QKV, O and down at 16.
struct GemvShape {
  int cb, w;
  bool staged;
};
constexpr int kGemvWavesPerCU = 12;
static GemvShape gemv_shape(const PackedWeight& w, int epi, int M, int ncu) {
  GemvShape sh;
  sh.cb = (epi == EPI_SWIGLU_F16 || epi == EPI_SWIGLU_F32) ? 2 : 1;
  const int KS = w.K / 64, groups = (w.N / 32 + sh.cb - 1) / sh.cb;
  const int D = (w.form == TGOHIP_FORM_I8 || w.form == TGOHIP_FORM_I4_TGO) ? 2 : 4;
  auto pick = [&](bool staged) {
    int wv = 0;
    for (int c : {4, 8, 16}) {
      if (staged && c == 4) continue;
      if (c > gemv_max_waves(w.form, sh.cb) || KS % (c * D) != 0) break;
      wv = c;
      if ((int64_t)groups * c >= (int64_t)kGemvWavesPerCU * ncu) break;
    }
    return wv;
  };
  // Staged when the rows fit and a staged wave count divides K; else direct.
  sh.staged = M <= 8 && (int64_t)M * gemv_stage_stride(w.K) * 2 <= kGemvStageBytes;
  sh.w = sh.staged ? pick(true) : 0;
  if (sh.w == 0) {
    sh.staged = false;
    sh.w = pick(false);
  }
  if (sh.w == 0 && KS % D == 0) sh.w = 1;
  return sh;
}

template <int FORM, int CB, int W, bool STAGED>
static void launch_gemv_w(const GemmArgs& g, int epi, hipStream_t st) {
  const dim3 grid((unsigned)((g.N / 32 + CB - 1) / CB)), blk(64 * W);
  const size_t lds = STAGED ? (size_t)g.M * gemv_stage_stride(g.K) * 2 : 0;
#define GEMV_LAUNCH(E, C)                                                                       \
  do {                                                                                          \
    if (STAGED) {                                                                               \
      static const hipError_t attr = hipFuncSetAttribute(                                        \
          (const void*)&gemm_gemv_kernel<FORM, E, C, W, STAGED>,                                 \
          hipFuncAttributeMaxDynamicSharedMemorySize, kGemvStageBytes);                          \
      (void)attr;                                                                               \
    }                                                                                           \
    hipLaunchKernelGGL((gemm_gemv_kernel<FORM, E, C, W, STAGED>), grid, blk, lds, st, g);      \
  } while (0)
  if constexpr (CB == 2) {
    if (epi == EPI_SWIGLU_F16) GEMV_LAUNCH(EPI_SWIGLU_F16, 2);
    else GEMV_LAUNCH(EPI_SWIGLU_F32, 2);
  } else {
    switch (epi) {
      case EPI_F32: GEMV_LAUNCH(EPI_F32, 1); break;
      case EPI_F16: GEMV_LAUNCH(EPI_F16, 1); break;
      default: GEMV_LAUNCH(EPI_RESID, 1); break;
    }
  }
#undef GEMV_LAUNCH
}

template <int FORM, int CB, bool STAGED>
static void launch_gemv_cb(const GemmArgs& g, int epi, int w, hipStream_t st) {
  switch (w) {  // the staged form runs 8 or 16 waves
    case 1: if constexpr (!STAGED) launch_gemv_w<FORM, CB, 1, STAGED>(g, epi, st); break;
    case 4: if constexpr (!STAGED) launch_gemv_w<FORM, CB, 4, STAGED>(g, epi, st); break;
    case 8: launch_gemv_w<FORM, CB, 8, STAGED>(g, epi, st); break;
    default:
      if constexpr (gemv_max_waves(FORM, CB) >= 16) launch_gemv_w<FORM, CB, 16, STAGED>(g, epi, st);
      break;
  }
}

template <int FORM>
static void launch_gemv_form(const GemmArgs& g, int epi, const GemvShape& sh, hipStream_t st) {
  if (sh.cb == 2) {
    if (sh.staged) launch_gemv_cb<FORM, 2, true>(g, epi, sh.w, st);
    else launch_gemv_cb<FORM, 2, false>(g, epi, sh.w, st);
  } else {
    if (sh.staged) launch_gemv_cb<FORM, 1, true>(g, epi, sh.w, st);
    else launch_gemv_cb<FORM, 1, false>(g, epi, sh.w, st);
  }
}

// The small-M kernels serve f16 activations up to 32 rows when K's k-steps
// divide into whole-depth shares.
static bool use_gemv(const PackedWeight& w, int xk, int M, int ncu) {
  return xk == XK_F16 && M <= 32 && w.form != TGOHIP_FORM_F16 &&
         gemv_shape(w, EPI_F32, M, ncu).w > 0;
}

// Split-K factor: enough workgroups to cover the chip twice, while each split
// keeps at least two 64-deep steps (a split past K's end computes zeros).
static int choose_splits(int M, int N, int K, int MW, int ncu) {
  const int tiles = ((N / 32 + 7) / 8) * ((M + MW - 1) / MW);
  const int KS = K / 64;
  int s = 1;
  while (tiles * s < 2 * ncu && KS / (s * 2) >= 2) s *= 2;
  return s;
}

// gemm_kernel's row tile: 32, 64 or 128 rows by M; 32 for a batch of at most
// 128 rows whose grid would not give every CU a workgroup (the C1 step, 67
// rows over f16 weights: 3.05 -> 2.05 ms per step with two-k-step splits).
static int small_mw(const PackedWeight& w, int M, int ncu) {
  const int mw = M <= 32 ? 32 : (M <= 64 ? 64 : 128);
  const int col_tiles = (w.N / 32 + 7) / 8;
  return (M <= 128 && col_tiles * ((M + mw - 1) / mw) < ncu) ? 32 : mw;
}

template <int FORM, int MW, bool ASPLIT>
static void launch_form(const GemmArgs& g, int epi, dim3 grid, hipStream_t st) {
  const dim3 blk(256);
  switch (epi) {
    case EPI_F32: hipLaunchKernelGGL((gemm_kernel<FORM, MW, ASPLIT, EPI_F32>), grid, blk, 0, st, g); break;
    case EPI_F16: hipLaunchKernelGGL((gemm_kernel<FORM, MW, ASPLIT, EPI_F16>), grid, blk, 0, st, g); break;
    case EPI_RESID: hipLaunchKernelGGL((gemm_kernel<FORM, MW, ASPLIT, EPI_RESID>), grid, blk, 0, st, g); break;
    case EPI_SWIGLU_F16: hipLaunchKernelGGL((gemm_kernel<FORM, MW, ASPLIT, EPI_SWIGLU_F16>), grid, blk, 0, st, g); break;
    case EPI_SWIGLU_F32: hipLaunchKernelGGL((gemm_kernel<FORM, MW, ASPLIT, EPI_SWIGLU_F32>), grid, blk, 0, st, g); break;
    case EPI_SWIGLU_X2:
      if constexpr (ASPLIT) hipLaunchKernelGGL((gemm_kernel<FORM, MW, ASPLIT, EPI_SWIGLU_X2>), grid, blk, 0, st, g);
      break;
  }
}

template <int MW, bool ASPLIT>
static void launch_mw(int form, const GemmArgs& g, int epi, dim3 grid, hipStream_t st) {
  switch (form) {
    case TGOHIP_FORM_F16: launch_form<TGOHIP_FORM_F16, MW, ASPLIT>(g, epi, grid, st); break;
    case TGOHIP_FORM_I8: launch_form<TGOHIP_FORM_I8, MW, ASPLIT>(g, epi, grid, st); break;
    case TGOHIP_FORM_I4_TGO: launch_form<TGOHIP_FORM_I4_TGO, MW, ASPLIT>(g, epi, grid, st); break;
    case TGOHIP_FORM_I4_SYM: launch_form<TGOHIP_FORM_I4_SYM, MW, ASPLIT>(g, epi, grid, st); break;
  }
}

static void launch_reduce(const GemmArgs& g, int epi, int splits, hipStream_t st) {
  const int outN = (epi == EPI_SWIGLU_F16 || epi == EPI_SWIGLU_F32 || epi == EPI_SWIGLU_X2) ? g.N / 2 : g.N;
  const size_t total = (size_t)g.M * outN;
  if (outN % 4 == 0 && g.pstride % 4 == 0) {  // four outputs per thread
    const dim3 rg4((unsigned)((total / 4 + 255) / 256)), rb4(256);
    switch (epi) {
      case EPI_F32: hipLaunchKernelGGL(gemm_reduce4_kernel<EPI_F32>, rg4, rb4, 0, st, g, splits); break;
      case EPI_F16: hipLaunchKernelGGL(gemm_reduce4_kernel<EPI_F16>, rg4, rb4, 0, st, g, splits); break;
      case EPI_RESID: hipLaunchKernelGGL(gemm_reduce4_kernel<EPI_RESID>, rg4, rb4, 0, st, g, splits); break;
      case EPI_SWIGLU_F16: hipLaunchKernelGGL(gemm_reduce4_kernel<EPI_SWIGLU_F16>, rg4, rb4, 0, st, g, splits); break;
      case EPI_SWIGLU_F32: hipLaunchKernelGGL(gemm_reduce4_kernel<EPI_SWIGLU_F32>, rg4, rb4, 0, st, g, splits); break;
      case EPI_SWIGLU_X2: hipLaunchKernelGGL(gemm_reduce4_kernel<EPI_SWIGLU_X2>, rg4, rb4, 0, st, g, splits); break;
    }
    return;
  }
  const dim3 rg((unsigned)((total + 255) / 256)), rb(256);
  switch (epi) {
    case EPI_F32: hipLaunchKernelGGL(gemm_reduce_kernel<EPI_F32>, rg, rb, 0, st, g, splits); break;
    case EPI_F16: hipLaunchKernelGGL(gemm_reduce_kernel<EPI_F16>, rg, rb, 0, st, g, splits); break;
    case EPI_RESID: hipLaunchKernelGGL(gemm_reduce_kernel<EPI_RESID>, rg, rb, 0, st, g, splits); break;
    case EPI_SWIGLU_F16: hipLaunchKernelGGL(gemm_reduce_kernel<EPI_SWIGLU_F16>, rg, rb, 0, st, g, splits); break;
    case EPI_SWIGLU_F32: hipLaunchKernelGGL(gemm_reduce_kernel<EPI_SWIGLU_F32>, rg, rb, 0, st, g, splits); break;
    case EPI_SWIGLU_X2: hipLaunchKernelGGL(gemm_reduce_kernel<EPI_SWIGLU_X2>, rg, rb, 0, st, g, splits); break;
  }
}

// Split-K factor for the pipelined kernel: none when the tiles fill at least
// half the chip's slots (2 per CU); otherwise as many splits as fit in one
// round of slots, keeping >= 8 k-steps per split.
// slots: workgroups the chip holds at once.
// TGOHIP_GEMM_MAX_SPLITS (1-8, default 8): the most split-K slices. At the
// C4 decode step (128 rows) a cap of 4 (fewer partial planes for QKV and O)
// or a rule keeping the planes' bytes below the weights' ran within the
// run-to-run spread of 8 over 4 alternating pairs of 300 steps (10.64-10.91
// against 10.62-10.65 ms); a cap of 2 was 5% slower.
static int pipe_max_splits() {
  static const int v = [] {
    const char* e = getenv("TGOHIP_GEMM_MAX_SPLITS");
    const int n = e ? atoi(e) : 8;
    return n >= 1 && n <= 8 ? n : 8;
  }();
  return v;
}

// TGOHIP_GEMM_EX_SPLITS (0: the rule below): split-K count for the exact
// (activation-pair) kernel's unsplit-by-rule launches other than SwiGLU.
static int pipe_ex_splits() {
  static const int v = [] {
    const char* e = getenv("TGOHIP_GEMM_EX_SPLITS");
    const int n = e ? atoi(e) : 0;
    return n >= 0 && n <= 8 ? n : 0;
  }();
  return v;
}

static int choose_pipe_splits(int tiles, int KS, int slots) {
  if (tiles <= 0 || tiles >= slots / 2) return 1;  // the partial sums would cost more than the fill gains
  int s = slots / tiles;              // one round of workgroups
  while (s > 1 && KS / s < 8) s--;
  return std::max(1, std::min(s, pipe_max_splits()));
}

// Row-tile height and split-K of the pipelined kernel. Up to 384 rows, 64-row
// tiles (3 workgroups per CU) waste fewer padded rows and give split-K more
// tiles to work with; above it, 128-row tiles (half the A re-reads and
// dequantization per MFMA) with split-K when they underfill the chip.
// Measured on the C3/C4 shapes: 64-row tiles without split-K lose to 128-row
// tiles with split-K at M = 1152, N = 4096.
// 128-row tiles go 8 waves wide (512 columns, one workgroup per CU) when the
// 512-column tiles deal evenly over the 8 XCDs: each activation tile read
// from L2 then feeds twice the columns (gate/up and down at M = 1152 measured
// 3-4% faster); otherwise 4 waves (256 columns, two workgroups per CU) keep
// the XCDs balanced (QKV, N = 6144: 12 wide tiles would leave four XCDs
// half idle, 45% slower).
// A SwiGLU epilogue needs whole sums, so a split gate/up goes through a
// separate reduction; with half the CUs covered by tiles it runs unsplit
// (at 128 rows: 45.6 us unsplit against 45.4 us plus a 7 us reduction).
// The exact (EX) kernel runs 64-row tiles 4 waves wide at every M: its A ring
// holds two planes, and at 128 rows its fragments would not fit the registers.
static void pipe_shape(const PackedWeight& w, int M, int ncu, int& mw, int& nw, int& tiles_n,
                       int& tiles, int& splits, int epi = EPI_F32, bool ex = false) {
  mw = (M <= 384 || ex) ? 64 : 128;
  const int nb = w.N / 32, rows = (M + mw - 1) / mw;
  nw = 4;
  if (mw == 128) {
    // 8 waves wide when the wide tiles deal evenly over the XCDs: over all 8
    // unsplit, or over the 8/s XCDs of a split when split-K slices them.
    const int tn8 = (nb + 15) / 16;
    const int s8 = choose_pipe_splits(tn8 * rows, w.K / 64, ncu);
    const int g8 = (s8 == 2 || s8 == 4 || s8 == 8) ? 8 / s8 : 8;
    if (tn8 % g8 == 0) nw = 8;
  }
  tiles_n = (nb + 2 * nw - 1) / (2 * nw);
  tiles = tiles_n * rows;
  splits = choose_pipe_splits(tiles, w.K / 64, ncu * (8 / nw));
  // The exact kernel's workgroups run three times the MFMAs, so an unsplit
  // launch's uneven last round costs more. Under 80% of one round of slots
  // it leaves most CUs one workgroup and the rest a second one: 4 splits
  // (the C4 O and down at 1152 rows, 288 tiles: 131 -> 118 and 377 -> 296 us
  // with the standalone reduction; the C5 O and down at 1280 rows, 400 tiles:
  // 342 -> 296 and 1011 -> 889 us in the step). One to 1.6 rounds: 2 splits
  // (the C5 QKV, 800 tiles: 404 -> 372 us). The C4 QKV (432 tiles, 84% of a
  // round) gained nothing from 2-5 splits and stays whole.
  if (ex && splits == 1) {
    const int slots = ncu * (8 / nw);
    if (5 * tiles < 4 * slots) splits = 4;
    else if (tiles > slots && 5 * tiles < 8 * slots) splits = 2;
    while (splits > 1 && (w.K / 64) / splits < 8) splits--;
  }
  if (ex && pipe_ex_splits() > 0) {
    splits = pipe_ex_splits();
    while (splits > 1 && (w.K / 64) / splits < 8) splits--;
  }
  // A SwiGLU launch over half the CUs or more stays whole (the reduction
  // would apply the epilogue), except an exact one under 80% of a round: the
  // C4 gate/up at 128 rows (192 tiles: whole, two k groups on 192 of 256
  // CUs) keeps the 2 splits of a launch under half the slots, with the
  // reduction, 74 -> 64.5 us (forced to 3, 4, 6 or 8 splits: 68-80 us).
  if ((epi == EPI_SWIGLU_F16 || epi == EPI_SWIGLU_F32 || epi == EPI_SWIGLU_X2) && tiles >= ncu / 2 &&
      !(ex && 5 * tiles < 4 * ncu * (8 / nw)))
    splits = 1;
}


template <int FORM, int MW, int NW, int KQ = 1, bool EX = false>
static void launch_pipe_form(const GemmArgs& g, int epi, dim3 grid, int tiles_n, int tiles,
                             int cm, int xs, const QKRopeArgs& qa, hipStream_t st) {
  const dim3 blk(64 * NW * KQ);
#define PIPE_LAUNCH(E) \
  hipLaunchKernelGGL((gemm_pipe_kernel<FORM, E, MW, NW, KQ, EX>), grid, blk, 0, st, g, tiles_n, tiles, cm, xs, qa)
  switch (epi) {
    case EPI_F32: PIPE_LAUNCH(EPI_F32); break;
    case EPI_F16: PIPE_LAUNCH(EPI_F16); break;
    case EPI_RESID: PIPE_LAUNCH(EPI_RESID); break;
    case EPI_SWIGLU_F16: if constexpr (!EX) PIPE_LAUNCH(EPI_SWIGLU_F16); break;
    case EPI_SWIGLU_F32: if constexpr (!EX) PIPE_LAUNCH(EPI_SWIGLU_F32); break;
    case EPI_SWIGLU_X2: if constexpr (EX) PIPE_LAUNCH(EPI_SWIGLU_X2); break;
    case EPI_QKROPE: if constexpr (EX && MW == 64 && NW == 4 && KQ == 1) PIPE_LAUNCH(EPI_QKROPE); break;
  }
#undef PIPE_LAUNCH
}

template <int FORM>
static void launch_pipe_shape(const GemmArgs& g, int epi, dim3 grid, int mw, int nw, int kq,
                              int tiles_n, int tiles, int cm, int xs, bool ex, const QKRopeArgs& qa,
                              hipStream_t st) {
  if (ex && kq == 2) launch_pipe_form<FORM, 64, 4, 2, true>(g, epi, grid, tiles_n, tiles, cm, xs, qa, st);
  else if (ex) launch_pipe_form<FORM, 64, 4, 1, true>(g, epi, grid, tiles_n, tiles, cm, xs, qa, st);
  else if (mw == 64 && kq == 2) launch_pipe_form<FORM, 64, 4, 2>(g, epi, grid, tiles_n, tiles, cm, xs, qa, st);
  else if (mw == 64) launch_pipe_form<FORM, 64, 4>(g, epi, grid, tiles_n, tiles, cm, xs, qa, st);
  else if (nw == 8) launch_pipe_form<FORM, 128, 8>(g, epi, grid, tiles_n, tiles, cm, xs, qa, st);
  else launch_pipe_form<FORM, 128, 4>(g, epi, grid, tiles_n, tiles, cm, xs, qa, st);
}

// TGOHIP_GEMM_KQ=0 keeps one k group in every workgroup.
static bool pipe_kq_enabled() {
  static const bool v = [] {
    const char* e = getenv("TGOHIP_GEMM_KQ");
    return !(e && atoi(e) == 0);
  }();
  return v;
}

// The pipelined kernel's launch: tile shape, k groups, k-steps per split and
// the split count those give.
struct PipeLaunch {
  int mw, nw, tiles_n, tiles, splits, kq, ksteps_per_split;
};
static PipeLaunch pipe_launch(const PackedWeight& w, int M, int ncu, int epi, bool ex) {
  PipeLaunch p;
  pipe_shape(w, M, ncu, p.mw, p.nw, p.tiles_n, p.tiles, p.splits, epi, ex);
  const int KS = w.K / 64;
  // Two k groups per workgroup (KQ = 2) where unsplit 64-row tiles would put
  // at most one wave on each SIMD (at most one workgroup per CU): the SwiGLU
  // gate/up of a 128-row step, 38.3 -> 35.6 us. Split projections keep one
  // group (O and down at 128 rows, 8 splits of 8 and 24 k-steps, ran 6% and
  // 2% slower with two).
  p.kq = (p.mw == 64 && p.splits == 1 && p.tiles <= ncu && KS % 8 == 0 && pipe_kq_enabled()) ? 2 : 1;
  // whole groups of 4 k-steps per split and k group (KS is a multiple of 4)
  p.ksteps_per_split = ((KS + p.splits - 1) / p.splits + 4 * p.kq - 1) / (4 * p.kq) * (4 * p.kq);
  p.splits = (KS + p.ksteps_per_split - 1) / p.ksteps_per_split;
  return p;
}

// xlo: the lo plane of an XK_X2 activation (the exact kernel), or null.
static int gemm_pipe_enqueue(const PackedWeight& w, const void* x, const void* xlo, int M, void* y,
                             int epi, float* workspace, size_t ws_bytes, int ncu, hipStream_t st,
                             int* defer, const QKRopeArgs* qa = nullptr) {
  const bool ex = xlo != nullptr;
  const PipeLaunch pl = pipe_launch(w, M, ncu, epi, ex);
  const int mw = pl.mw, nw = pl.nw, tiles_n = pl.tiles_n, tiles = pl.tiles, kq = pl.kq;
  int splits = pl.splits;
  GemmArgs g{};
  g.x = x;
  g.xlo = xlo;
  g.wp = w.wp;
  g.ws = w.ws;
  g.wz = w.wz;
  g.y = y;
  g.M = M;
  g.K = w.K;
  g.N = w.N;
  g.ksteps_per_split = pl.ksteps_per_split;
  if (splits > 1) {
    if (!workspace || ws_bytes < (size_t)splits * split_plane_stride(M, w.N) * sizeof(float))
      return fail(TGOHIP_ESTATE, "linear: split-K workspace too small");
    g.part = workspace;
    g.pstride = split_plane_stride(M, w.N);
  }
  // 2, 4 or 8 splits slice the XCDs (see the kernel), others ride grid.z.
  const int xs = (splits == 2 || splits == 4 || splits == 8) ? splits : 0;
  const int G = xs ? 8 / xs : 8;
  const dim3 grid((unsigned)(8 * ((tiles_n + G - 1) / G) * (tiles / tiles_n)), 1,
                  (unsigned)(xs ? 1 : splits));
  // Few row tiles (at most 4: the LM head at a batch's 130-odd rows): the row
  // tiles of a column tile run side by side and read its weights once
  // (262 -> 250 us for the C4 LM head at 136 rows).
  const int cm = tiles / tiles_n <= 4 ? 1 : 0;
  switch (w.form) {
    case TGOHIP_FORM_I4_SYM:
      launch_pipe_shape<TGOHIP_FORM_I4_SYM>(g, epi, grid, mw, nw, kq, tiles_n, tiles, cm, xs, ex, qa ? *qa : QKRopeArgs{}, st);
      break;
    case TGOHIP_FORM_I4_TGO:
      launch_pipe_shape<TGOHIP_FORM_I4_TGO>(g, epi, grid, mw, nw, kq, tiles_n, tiles, cm, xs, ex, qa ? *qa : QKRopeArgs{}, st);
      break;
    default:
      launch_pipe_shape<TGOHIP_FORM_I8>(g, epi, grid, mw, nw, kq, tiles_n, tiles, cm, xs, ex, qa ? *qa : QKRopeArgs{}, st);
      break;
  }
  if (defer) *defer = splits > 1 ? splits : 0;
  if (splits > 1 && !defer) launch_reduce(g, epi, splits, st);
  TGOHIP_HIP(hipGetLastError());
  return 0;
}

// The pipelined kernel serves f16 activations from this many rows up (below
// it the small-M kernel; at 48-80 rows the pipelined kernel measured 10-30%
// faster than gemm_kernel for the int4 packs).
static int pipe_min_rows() {
  static const int v = [] {
    const char* e = getenv("TGOHIP_GEMM_PIPE_MIN");
    return e ? atoi(e) : 33;
  }();
  return v;
}

// The pipelined kernel serves the int4 packs and int8 with f16 activations
// or activation pairs (XK_X2, the exact kernel); f16 weights and unsplit f32
// activations use gemm_kernel.
static bool use_pipe(const PackedWeight& w, int xk, int M) {
  return xk != XK_F32 && w.form != TGOHIP_FORM_F16 && M >= pipe_min_rows() &&
         (w.K / 64) % 4 == 0 &&
         (int64_t)M * w.K < ((int64_t)1 << 31);  // its activation offsets are 32-bit
}

// Workspace bytes a call needs for split-K partials: xk < 0 bounds every
// activation type and epilogue; otherwise the bytes of exactly the call
// gemm_enqueue makes over that activation type with an f32 or f16 epilogue.
size_t gemm_workspace_bytes(const PackedWeight& w, int M, int ncu, int xk) {
  if (M <= 0) return 0;  // nothing launches (and no tiles to divide the slots by)
  const int MW = small_mw(w, M, ncu);
  int s;
  if (xk < 0) {
    s = std::max({choose_splits(M, w.N, w.K, MW, ncu), pipe_launch(w, M, ncu, EPI_F32, false).splits,
                  pipe_launch(w, M, ncu, EPI_F32, true).splits});
  } else if (use_pipe(w, xk, M)) {
    s = pipe_launch(w, M, ncu, EPI_F32, xk == XK_X2).splits;
  } else if (use_gemv(w, xk, M, ncu)) {
    s = 1;
  } else {
    s = choose_splits(M, w.N, w.K, MW, ncu);  // gemm_kernel's grid.z
  }
  return s > 1 ? (size_t)s * split_plane_stride(M, w.N) * sizeof(float) : 0;
}

// The QKV projection with q/k-norm, RoPE and the K/V write in its epilogue
// (EPI_QKROPE): an activation pair on the pipelined exact kernel, unsplit,
// one k group per workgroup, whole 128-wide heads in each 256-column tile,
// and a rope table for the rows.
bool gemm_qkrope_fusable(const PackedWeight& w, int M, int ncu) {
  if (M <= 0 || !use_pipe(w, XK_X2, M) || w.N % 256 != 0) return false;
  const PipeLaunch pl = pipe_launch(w, M, ncu, EPI_F32, true);
  return pl.splits == 1 && pl.kq == 1 && pl.mw == 64 && pl.nw == 4;
}

int gemm_enqueue_qkrope(const PackedWeight& w, const void* x, int M, const QKRopeArgs& qa, int ncu,
                        hipStream_t st) {
  if (!gemm_qkrope_fusable(w, M, ncu) || !qa.rope || w.N != (qa.H + 2 * qa.Hkv) * 128)
    return fail(TGOHIP_ESTATE, "linear: the fused QKV epilogue does not apply to this launch");
  const void* xlo = (const half_t*)x + (size_t)M * w.K;
  return gemm_pipe_enqueue(w, x, xlo, M, nullptr, EPI_QKROPE, nullptr, 0, ncu, st, nullptr, &qa);
}

int gemm_enqueue(const PackedWeight& w, const void* x, int xk, int M, void* y, int epi,
                 float* workspace, size_t ws_bytes, int ncu, hipStream_t st, int* defer) {
  if (defer) *defer = 0;
  if (M <= 0) return 0;
  if (defer && epi != EPI_F32 && epi != EPI_RESID)
    return fail(TGOHIP_ESTATE, "linear: only f32 and residual epilogues can defer split-K");
  // a SwiGLU over activation-pair input stores a pair, and only then
  if (xk == XK_X2 ? (epi == EPI_SWIGLU_F16 || epi == EPI_SWIGLU_F32) : epi == EPI_SWIGLU_X2)
    return fail(TGOHIP_ESTATE, "linear: the activation-pair SwiGLU output goes with activation-pair input");
  // an activation pair's lo plane follows its hi plane
  const void* xlo = xk == XK_X2 ? (const void*)((const half_t*)x + (size_t)M * w.K) : nullptr;
  if (use_pipe(w, xk, M))
    return gemm_pipe_enqueue(w, x, xlo, M, y, epi, workspace, ws_bytes, ncu, st, defer);
  if (use_gemv(w, xk, M, ncu)) {
    GemmArgs g{};
    g.x = x;
    g.wp = w.wp;
    g.ws = w.ws;
    g.wz = w.wz;
    g.y = y;
    g.M = M;
    g.K = w.K;
    g.N = w.N;
    const GemvShape sh = gemv_shape(w, epi, M, ncu);
    switch (w.form) {
      case TGOHIP_FORM_F16: launch_gemv_form<TGOHIP_FORM_F16>(g, epi, sh, st); break;
      case TGOHIP_FORM_I8: launch_gemv_form<TGOHIP_FORM_I8>(g, epi, sh, st); break;
      case TGOHIP_FORM_I4_TGO: launch_gemv_form<TGOHIP_FORM_I4_TGO>(g, epi, sh, st); break;
      case TGOHIP_FORM_I4_SYM: launch_gemv_form<TGOHIP_FORM_I4_SYM>(g, epi, sh, st); break;
    }
    TGOHIP_HIP(hipGetLastError());
    return 0;
  }
  const int MW = small_mw(w, M, ncu);
  const int splits = choose_splits(M, w.N, w.K, MW, ncu);
  const bool split_a = xk != XK_F16;  // f32 or an activation pair: hi + lo planes
  GemmArgs g{};
  g.x = x;
  g.xlo = xlo;
  g.wp = w.wp;
  g.ws = w.ws;
  g.wz = w.wz;
  g.y = y;
  g.M = M;
  g.K = w.K;
  g.N = w.N;
  const int KS = w.K / 64;
  g.ksteps_per_split = (KS + splits - 1) / splits;
  if (splits > 1) {
    if (!workspace || ws_bytes < (size_t)splits * split_plane_stride(M, w.N) * sizeof(float))
      return fail(TGOHIP_ESTATE, "linear: split-K workspace too small");
    g.part = workspace;
    g.pstride = split_plane_stride(M, w.N);
  }
  const dim3 grid((unsigned)((w.N / 32 + 7) / 8), (unsigned)((M + MW - 1) / MW), (unsigned)splits);
  if (MW == 32) {
    if (split_a) launch_mw<32, true>(w.form, g, epi, grid, st);
    else launch_mw<32, false>(w.form, g, epi, grid, st);
  } else if (MW == 64) {
    if (split_a) launch_mw<64, true>(w.form, g, epi, grid, st);
    else launch_mw<64, false>(w.form, g, epi, grid, st);
  } else {
    if (split_a) launch_mw<128, true>(w.form, g, epi, grid, st);
    else launch_mw<128, false>(w.form, g, epi, grid, st);
  }
  if (defer) *defer = splits > 1 ? splits : 0;
  if (splits > 1 && !defer) launch_reduce(g, epi, splits, st);
  TGOHIP_HIP(hipGetLastError());
  return 0;
}

}  // namespace tgohip
