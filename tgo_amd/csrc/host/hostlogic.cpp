// hostlogic.cpp -- host-side mirrors of tgo's batched path that run on the
// CPU: model.NewBatchStep (model/batch.go), nextStep/victim (schedule.go),
// the weight conversions of weights/convert.go, and the prefix block pool
// (internal/prefix). Same names, argument meaning and refusals as the Go.
#include <stdint.h>
#include <string.h>
#include <math.h>

#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "../../../include/tgohip.h"
#include "hostlogic.h"

namespace tgohip {
int fail(int code, const std::string& msg);
}
using tgohip::fail;

// ---------------------------------------------------------------------------
// weights/convert.go
// ---------------------------------------------------------------------------
static uint32_t round_shift(uint32_t v, uint32_t n) {
  if (n == 0) return v;
  uint32_t keep = v >> n, rest = v & ((1u << n) - 1), half = 1u << (n - 1);
  if (rest > half || (rest == half && (keep & 1))) keep++;
  return keep;
}

// f32ToF16Bits (weights/convert.go:153-180).
uint16_t tgohip_f16_bits(float x, int* saturated) {
  uint32_t b;
  memcpy(&b, &x, 4);
  const uint16_t sign = (uint16_t)((b >> 16) & 0x8000);
  if (saturated) *saturated = 0;
  if ((b & 0x7fffffffu) > 0x7f800000u) return 0x7e00;
  uint32_t ab = b & 0x7fffffffu;
  float a;
  memcpy(&a, &ab, 4);
  if (a > 65504.0f) {
    if (saturated) *saturated = 1;
    return sign | 0x7bff;
  }
  if (a < 1.0f / 16384.0f) return sign;
  const int32_t e = (int32_t)((b >> 23) & 0xff) - 127;
  const uint32_t mant = b & 0x7fffffu;
  return (uint16_t)(sign | (uint16_t)(((uint32_t)(e + 15) << 10) + round_shift(mant, 13)));
}

static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  uint32_t u;
  if (e == 0) {
    if (m == 0) { u = sign; float f; memcpy(&f, &u, 4); return f; }
    const float v = ldexpf((float)m, -24);
    return (h & 0x8000) ? -v : v;
  }
  if (e == 31) u = sign | 0x7f800000u | (m << 13);
  else u = sign | ((e + 112) << 23) | (m << 13);
  float f;
  memcpy(&f, &u, 4);
  return f;
}

extern "C" size_t tgohip_to_f16(const float* src, uint16_t* dst, size_t n) {
  size_t sat = 0;
  for (size_t i = 0; i < n; i++) {
    int s;
    dst[i] = tgohip_f16_bits(src[i], &s);
    sat += (size_t)s;
  }
  return sat;
}

// quantizeInto (weights/convert.go:206-217): per 32 flattened elements, scale
// f16(peak/127), q = round-half-even(x / scale) clamped to [-127, 127].
extern "C" void tgohip_quantize_int8(const float* w, size_t n, int8_t* q, uint16_t* scales) {
  for (size_t lo = 0; lo < n; lo += 32) {
    const size_t hi = std::min(lo + 32, n);
    float peak = 0;
    for (size_t i = lo; i < hi; i++) peak = std::max(peak, fabsf(w[i]));
    const uint16_t s16 = tgohip_f16_bits(peak / 127.0f, nullptr);
    const float s = f16_to_f32(s16);
    scales[lo / 32] = s16;
    for (size_t i = lo; i < hi; i++) {
      double v = s > 0 ? nearbyint((double)w[i] / (double)s) : 0.0;
      v = std::max(-127.0, std::min(127.0, v));
      q[i] = (int8_t)v;
    }
  }
}

// The int4 triple of nn.FormInt4 (nn/nn.go:128-135; weights/weights.go:694-743):
// per 128 flattened elements, s = f16((max-min)/15), z = an integer in [0,15]
// as f16, q = clamp(round-half-even(x/s + z), 0, 15), 8 codes per u32 word,
// element i of a word in bits 4i..4i+3.
extern "C" void tgohip_quantize_int4(const float* w, size_t n, uint32_t* codes, uint16_t* scales,
                                     uint16_t* zeros) {
  memset(codes, 0, (n + 7) / 8 * 4);
  for (size_t lo = 0; lo < n; lo += 128) {
    const size_t hi = std::min(lo + 128, n);
    float mn = w[lo], mx = w[lo];
    for (size_t i = lo; i < hi; i++) { mn = std::min(mn, w[i]); mx = std::max(mx, w[i]); }
    const float sr = (mx - mn) / 15.0f;
    uint16_t s16 = tgohip_f16_bits(sr > 0 ? sr : 1.0f, nullptr);
    float s = f16_to_f32(s16);
    if (s == 0) { s16 = 0x3c00; s = 1.0f; }
    double zf = nearbyint(-(double)mn / (double)s);
    zf = std::max(0.0, std::min(15.0, zf));
    scales[lo / 128] = s16;
    zeros[lo / 128] = tgohip_f16_bits((float)zf, nullptr);
    for (size_t i = lo; i < hi; i++) {
      double v = nearbyint((double)w[i] / (double)s + zf);
      v = std::max(0.0, std::min(15.0, v));
      codes[i / 8] |= ((uint32_t)v & 15u) << (4 * (i % 8));
    }
  }
}

// ---------------------------------------------------------------------------
// model/batch.go:66-152 -- NewBatchStep
// ---------------------------------------------------------------------------
extern "C" int tgohip_new_batch_step(int vocab, int heads, int kv_heads, int rows, int B,
                                     const int32_t* tokens, const int32_t* counts,
                                     const int32_t* first, const int32_t* pages,
                                     const int32_t* pages_len, int max_pages, int block,
                                     int capacity, uint32_t* ids, uint32_t* posq, uint32_t* posk,
                                     uint32_t* slots, uint32_t* lengths, uint32_t* extents,
                                     uint32_t* last) {
  if (B < 2)
    return fail(TGOHIP_EINVAL, "NewBatchStep: " + std::to_string(B) +
                                   " member(s); a batch is two or more sequences, and one is NewStep");
  if (block <= 0)
    return fail(TGOHIP_EINVAL, "NewBatchStep: block is " + std::to_string(block) +
                                   "; sequences that step together are addressed through a page table");
  int64_t total = 0;
  for (int i = 0; i < B; i++) total += counts[i];
  if (total == 0)
    return fail(TGOHIP_EINVAL, "NewBatchStep: every member contributes nothing; a step with no "
                               "rows computes nothing and has no logits to read");
  if (total > rows)
    return fail(TGOHIP_EINVAL, "NewBatchStep: " + std::to_string(total) +
                                   " member tokens do not fit a " + std::to_string(rows) + "-row plan");
  int at = 0, pad = -1;
  int64_t tokoff = 0;
  std::vector<int64_t> off(B);
  for (int i = 0; i < B; i++) { off[i] = tokoff; tokoff += counts[i]; }
  for (int i = 0; i < B; i++) {
    lengths[i] = (uint32_t)(first[i] + counts[i]);
    extents[i] = (uint32_t)counts[i];
    last[i] = 0;
    if (first[i] < 0)
      return fail(TGOHIP_EINVAL, "NewBatchStep: member " + std::to_string(i) + " starts at position " +
                                     std::to_string(first[i]) + "; a position is not negative");
    if (counts[i] > 0) {
      pad = i;
      last[i] = (uint32_t)(at + counts[i] - 1);
    }
    for (int j = 0; j < counts[i]; j++) {
      const int id = tokens[off[i] + j];
      if (id < 0 || id >= vocab)
        return fail(TGOHIP_EINVAL, "NewBatchStep: member " + std::to_string(i) + " token id " +
                                       std::to_string(id) + " is outside the model's vocabulary of " +
                                       std::to_string(vocab));
      const int p = first[i] + j;
      const int need = p / block + 1;
      if (need > pages_len[i])
        return fail(TGOHIP_EINVAL, "NewBatchStep: member " + std::to_string(i) + " reaches position " +
                                       std::to_string(p) + ", which needs " + std::to_string(need) +
                                       " page table entries and it has " + std::to_string(pages_len[i]) +
                                       "; the missing block is one another sequence owns");
      ids[at] = (uint32_t)id;
      slots[at] = (uint32_t)(pages[(size_t)i * max_pages + p / block] * block + p % block);
      for (int h = 0; h < heads; h++) posq[(size_t)at * heads + h] = (uint32_t)p;
      for (int h = 0; h < kv_heads; h++) posk[(size_t)at * kv_heads + h] = (uint32_t)p;
      at++;
    }
  }
  // The padding: the last real token at its position, slot = capacity.
  if (at < rows && pad >= 0) {
    const uint32_t lastTok = (uint32_t)tokens[off[pad] + counts[pad] - 1];
    const uint32_t lastPos = (uint32_t)(first[pad] + counts[pad] - 1);
    for (; at < rows; at++) {
      ids[at] = lastTok;
      slots[at] = (uint32_t)capacity;
      for (int h = 0; h < heads; h++) posq[(size_t)at * heads + h] = lastPos;
      for (int h = 0; h < kv_heads; h++) posk[(size_t)at * kv_heads + h] = lastPos;
    }
  }
  return 0;
}

// ---------------------------------------------------------------------------
// schedule.go:80-150 -- nextStep, victim
// ---------------------------------------------------------------------------
extern "C" int tgohip_next_step(int n, const int32_t* live, const int32_t* prompt_len,
                                const int32_t* prefilled, int chunk, int rows, int32_t* work_slot,
                                int32_t* work_start, int32_t* work_count, int32_t* n_work,
                                int32_t* prefill, int32_t* decode) {
  if (chunk <= 0)
    return fail(TGOHIP_EINVAL, "the prefill chunk is " + std::to_string(chunk) +
                                   "; a chunk is at least one token");
  if (rows <= 0)
    return fail(TGOHIP_EINVAL, "a step of " + std::to_string(rows) + " rows carries nothing");
  struct W { int slot, start, count; };
  std::vector<W> work;
  int left = rows, pf = 0, dc = 0;
  for (int i = 0; i < n; i++) {
    if (!live[i] || prefilled[i] >= prompt_len[i]) continue;
    const int c = std::min(std::min(chunk, prompt_len[i] - prefilled[i]), left);
    if (c <= 0) continue;
    work.push_back({i, prefilled[i], c});
    pf += c;
    left -= c;
  }
  for (int i = 0; i < n; i++) {
    if (!live[i] || prefilled[i] < prompt_len[i] || left <= 0) continue;
    work.push_back({i, -1, 1});
    dc++;
    left--;
  }
  std::stable_sort(work.begin(), work.end(), [](const W& a, const W& b) { return a.slot < b.slot; });
  for (size_t i = 0; i < work.size(); i++) {
    work_slot[i] = work[i].slot;
    work_start[i] = work[i].start;
    work_count[i] = work[i].count;
  }
  *n_work = (int32_t)work.size();
  *prefill = pf;
  *decode = dc;
  return 0;
}

extern "C" int tgohip_victim(int n, const int32_t* live, const int32_t* prompt_len,
                             const int32_t* prefilled, const uint64_t* arrived) {
  int best = -1;
  uint64_t bestKey = 0;
  for (int i = 0; i < n; i++) {
    if (!live[i]) continue;
    uint64_t key = arrived[i];
    if (prefilled[i] < prompt_len[i]) key |= 1ull << 63;
    if (best < 0 || key > bestKey) { best = i; bestKey = key; }
  }
  return best;
}

// ---------------------------------------------------------------------------
// SHA-256 (FIPS 180-4), for the prefix hash chain (internal/prefix/hash.go)
// ---------------------------------------------------------------------------
namespace {
struct Sha256 {
  uint32_t h[8];
  uint8_t buf[64];
  uint64_t len = 0;
  size_t fill = 0;
  Sha256() {
    static const uint32_t init[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                     0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    memcpy(h, init, sizeof(h));
  }
  static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
  void block(const uint8_t* p) {
    static const uint32_t k[64] = {
        0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
        0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
        0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
        0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
        0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
        0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
        0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
        0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
    uint32_t w[64];
    for (int i = 0; i < 16; i++)
      w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
    for (int i = 16; i < 64; i++) {
      const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
      const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
      w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int i = 0; i < 64; i++) {
      const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
      const uint32_t ch = (e & f) ^ (~e & g);
      const uint32_t t1 = hh + S1 + ch + k[i] + w[i];
      const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
      const uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
      const uint32_t t2 = S0 + mj;
      hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
  }
  void update(const void* data, size_t n) {
    const uint8_t* p = (const uint8_t*)data;
    len += n;
    while (n > 0) {
      const size_t take = std::min(n, 64 - fill);
      memcpy(buf + fill, p, take);
      fill += take;
      p += take;
      n -= take;
      if (fill == 64) { block(buf); fill = 0; }
    }
  }
  void digest(uint8_t out[32]) {
    const uint64_t bits = len * 8;
    const uint8_t one = 0x80, zero = 0;
    update(&one, 1);
    while (fill != 56) update(&zero, 1);
    uint8_t lb[8];
    for (int i = 0; i < 8; i++) lb[i] = (uint8_t)(bits >> (56 - 8 * i));
    update(lb, 8);
    for (int i = 0; i < 8; i++) {
      out[4 * i] = (uint8_t)(h[i] >> 24);
      out[4 * i + 1] = (uint8_t)(h[i] >> 16);
      out[4 * i + 2] = (uint8_t)(h[i] >> 8);
      out[4 * i + 3] = (uint8_t)h[i];
    }
  }
};
void put_u64(Sha256& s, uint64_t v) {
  uint8_t b[8];
  for (int i = 0; i < 8; i++) b[i] = (uint8_t)(v >> (8 * i));
  s.update(b, 8);
}
}  // namespace

// seed (internal/prefix/hash.go:28-42)
Hash32 prefix_seed(int scope, const std::string& domain, const std::string& salt) {
  Sha256 s;
  s.update("tgo/prefix/v1", 13);
  put_u64(s, (uint64_t)(int64_t)scope);
  for (const std::string* f : {&domain, &salt}) {
    put_u64(s, f->size());
    s.update(f->data(), f->size());
  }
  Hash32 out;
  s.digest(out.b);
  return out;
}
// chain (internal/prefix/hash.go:54-65)
Hash32 prefix_chain(const Hash32& prev, const int32_t* ids, int n) {
  Sha256 s;
  s.update(prev.b, 32);
  for (int i = 0; i < n; i++) put_u64(s, (uint64_t)(int64_t)ids[i]);
  Hash32 out;
  s.digest(out.b);
  return out;
}

extern "C" int tgohip_sha256(const void* data, size_t n, uint8_t* out32) {
  Sha256 s;
  s.update(data, n);
  s.digest(out32);
  return 0;
}

// ---------------------------------------------------------------------------
// internal/prefix/prefix.go, lease.go
// ---------------------------------------------------------------------------
PrefixPool::PrefixPool(int block_, int blocks_, int scope_)
    : block(block_), blocks(blocks_), scope(scope_), blk(blocks_), head(-1), tail(-1) {
  free.resize(blocks);
  for (int i = 0; i < blocks; i++) free[i] = blocks - 1 - i;  // low index handed out first
  st.free = blocks;
}

void PrefixPool::lru_push(int id) {
  Blk& b = blk[id];
  b.prev = tail;
  b.next = -1;
  if (tail >= 0) blk[tail].next = id;
  else head = id;
  tail = id;
}
void PrefixPool::lru_remove(int id) {
  Blk& b = blk[id];
  if (b.prev >= 0) blk[b.prev].next = b.next;
  else head = b.next;
  if (b.next >= 0) blk[b.next].prev = b.prev;
  else tail = b.prev;
  b.prev = b.next = -1;
}
void PrefixPool::evict(int id) {
  Blk& b = blk[id];
  lru_remove(id);
  entry.erase(b.hash);
  b.hash = Hash32();
  b.published = false;
  st.cached--;
  st.evictions++;
}
bool PrefixPool::take(int& out) {
  if (!free.empty()) {
    out = free.back();
    free.pop_back();
    st.free--;
    blk[out].refs = 1;
    st.in_use++;
    return true;
  }
  if (head < 0) return false;
  out = head;
  evict(out);
  blk[out].refs = 1;
  st.in_use++;
  return true;
}
void PrefixPool::hold(int id) {
  Blk& b = blk[id];
  b.refs++;
  if (b.refs == 1) {
    lru_remove(id);
    st.cached--;
    st.in_use++;
  }
}
void PrefixPool::drop(int id) {
  Blk& b = blk[id];
  b.refs--;
  if (b.refs > 0) return;
  st.in_use--;
  if (b.published) {
    lru_push(id);
    st.cached++;
    return;
  }
  free.push_back(id);
  st.free++;
}
void PrefixPool::release_taken(int id) {
  blk[id].refs = 0;
  st.in_use--;
  free.push_back(id);
  st.free++;
}
int PrefixPool::alloc(int n, std::vector<int>& out) {
  std::vector<int> got;
  while ((int)got.size() < n) {
    int id;
    if (!take(id)) {
      for (int g : got) release_taken(g);
      return fail(TGOHIP_EEXHAUSTED, "prefix: " + std::to_string(st.in_use) + " of " +
                                         std::to_string(blocks) +
                                         " blocks are referenced by a live sequence: prefix: the block pool is exhausted");
    }
    got.push_back(id);
  }
  out.insert(out.end(), got.begin(), got.end());
  return 0;
}

int PrefixPool::acquire(const int32_t* ids, int n, const std::string& session,
                        const std::string& salt, int reserve, PrefixLease** out) {
  if (n <= 0) return fail(TGOHIP_EINVAL, "prefix: the prompt is empty; there is no prefix to key on");
  if (scope == 1 && session.empty())
    return fail(TGOHIP_EINVAL, "prefix: the scope is session and the request names no session; "
                               "an unnamed session would share with every other unnamed one");
  if (reserve < 0)
    return fail(TGOHIP_EINVAL, "prefix: the reserve is " + std::to_string(reserve) +
                                   "; it is positions to hold beyond the prompt");
  const int need = (n + reserve + block - 1) / block;
  if (need > blocks)
    return fail(TGOHIP_EEXHAUSTED, "prefix: a " + std::to_string(n) + "-token prompt with a reserve of " +
                                       std::to_string(reserve) + " needs " + std::to_string(need) +
                                       " blocks and the pool holds " + std::to_string(blocks) +
                                       ": prefix: the block pool is exhausted");
  PrefixLease* l = new PrefixLease();
  l->pool = this;
  l->ids.assign(ids, ids + n);
  l->seed = prefix_seed(scope, scope == 1 ? session : std::string(), salt);
  if (scope != 2) {
    Hash32 prev = l->seed;
    for (int i = 0; i < n / block; i++) {
      prev = prefix_chain(prev, ids + (size_t)i * block, block);
      l->hashes.push_back(prev);
    }
  }
  int matched = 0;
  const int limit = (n - 1) / block;
  while (matched < limit && matched < (int)l->hashes.size()) {
    auto it = entry.find(l->hashes[matched]);
    if (it == entry.end()) break;
    hold(it->second);
    l->blocks.push_back(it->second);
    matched++;
  }
  std::vector<int> fresh;
  if (alloc(need - matched, fresh) != 0) {
    for (int b : l->blocks) drop(b);
    delete l;
    return TGOHIP_EEXHAUSTED;
  }
  l->blocks.insert(l->blocks.end(), fresh.begin(), fresh.end());
  l->matched = matched;
  l->reused = matched * block;
  l->published = matched;
  st.acquires++;
  st.prompt += n;
  st.reused += l->reused;
  if (matched > 0) st.hits++;
  *out = l;
  return 0;
}

int PrefixLease::grow(int n) {
  if (released) return fail(TGOHIP_ESTATE, "prefix: the lease is released");
  if (n < 0) return fail(TGOHIP_EINVAL, "prefix: growing by " + std::to_string(n) + " positions");
  if (n == 0) return 0;
  const int want = ((int)ids.size() + n + pool->block - 1) / pool->block;
  if (want > pool->blocks)
    return fail(TGOHIP_EEXHAUSTED, "prefix: " + std::to_string(ids.size() + n) + " positions need " +
                                       std::to_string(want) + " blocks and the pool holds " +
                                       std::to_string(pool->blocks) + ": prefix: the block pool is exhausted");
  const int k = want - (int)blocks.size();
  if (k > 0) {
    std::vector<int> fresh;
    if (pool->alloc(k, fresh) != 0) return TGOHIP_EEXHAUSTED;
    blocks.insert(blocks.end(), fresh.begin(), fresh.end());
  }
  return 0;
}

int PrefixLease::commit(const int32_t* add, int n) {
  if (released) return fail(TGOHIP_ESTATE, "prefix: the lease is released");
  if (n == 0) return 0;
  const int want = ((int)ids.size() + n + pool->block - 1) / pool->block;
  if (want > (int)blocks.size())
    return fail(TGOHIP_EINVAL, "prefix: committing " + std::to_string(n) + " tokens at position " +
                                   std::to_string(ids.size()) + " needs " + std::to_string(want) +
                                   " blocks and the lease holds " + std::to_string(blocks.size()) +
                                   "; grow it before the step that computes them");
  ids.insert(ids.end(), add, add + n);
  if (pool->scope != 2) {
    Hash32 prev = hashes.empty() ? seed : hashes.back();
    for (int i = (int)hashes.size(); i < (int)ids.size() / pool->block; i++) {
      prev = prefix_chain(prev, ids.data() + (size_t)i * pool->block, pool->block);
      hashes.push_back(prev);
    }
  }
  return 0;
}

void PrefixLease::publish(int written) {
  if (released || pool->scope == 2) return;
  const int complete = written / pool->block;
  for (int i = published; i < (int)hashes.size() && i < complete; i++) {
    const Hash32& h = hashes[i];
    const int mine = blocks[i];
    auto it = pool->entry.find(h);
    if (it != pool->entry.end()) {
      const int theirs = it->second;
      if (theirs != mine) {
        pool->hold(theirs);
        pool->drop(mine);
        blocks[i] = theirs;
        pool->st.adoptions++;
      }
      published = i + 1;
      continue;
    }
    pool->entry[h] = mine;
    pool->blk[mine].hash = h;
    pool->blk[mine].published = true;
    pool->st.publishes++;
    published = i + 1;
  }
}

void PrefixLease::release() {
  if (released) return;
  released = true;
  for (int b : blocks) pool->drop(b);
}

// C ABI over the pool.
struct tgohip_pool { PrefixPool p; tgohip_pool(int a, int b, int c) : p(a, b, c) {} };
struct tgohip_lease { PrefixLease* l; };

extern "C" tgohip_pool* tgohip_pool_new(int block, int blocks, int scope) {
  if (block <= 0) { fail(TGOHIP_EINVAL, "prefix: the block size is " + std::to_string(block) + "; a block holds at least one position"); return nullptr; }
  if (blocks <= 0) { fail(TGOHIP_EINVAL, "prefix: the pool holds " + std::to_string(blocks) + " blocks; a pool holds at least one"); return nullptr; }
  if (scope < 0 || scope > 2) { fail(TGOHIP_EINVAL, "prefix: scope(" + std::to_string(scope) + ") is not a scope"); return nullptr; }
  return new tgohip_pool(block, blocks, scope);
}
extern "C" void tgohip_pool_free(tgohip_pool* p) { delete p; }
extern "C" void tgohip_pool_stats(tgohip_pool* p, int64_t* s) {
  const PrefixStats& t = p->p.st;
  const int64_t v[10] = {t.acquires, t.hits, t.reused, t.prompt, t.evictions, t.publishes,
                         t.adoptions, t.in_use, t.cached, t.free};
  memcpy(s, v, sizeof(v));
}
extern "C" int tgohip_pool_acquire(tgohip_pool* p, const int32_t* ids, int n, const char* session,
                                   const char* salt, int reserve, tgohip_lease** out) {
  PrefixLease* l = nullptr;
  const int rc = p->p.acquire(ids, n, session ? session : "", salt ? salt : "", reserve, &l);
  if (rc != 0) return rc;
  *out = new tgohip_lease{l};
  return 0;
}
extern "C" int tgohip_lease_blocks(tgohip_lease* l, int32_t* out, int cap) {
  const int n = (int)l->l->blocks.size();
  for (int i = 0; i < n && i < cap; i++) out[i] = l->l->blocks[i];
  return n;
}
extern "C" int tgohip_lease_reused(tgohip_lease* l) { return l->l->reused; }
extern "C" int tgohip_lease_len(tgohip_lease* l) { return (int)l->l->ids.size(); }
extern "C" int tgohip_lease_grow(tgohip_lease* l, int n) { return l->l->grow(n); }
extern "C" int tgohip_lease_commit(tgohip_lease* l, const int32_t* ids, int n) { return l->l->commit(ids, n); }
extern "C" int tgohip_lease_publish(tgohip_lease* l, int written) { l->l->publish(written); return 0; }
extern "C" void tgohip_lease_release(tgohip_lease* l) { l->l->release(); }
extern "C" void tgohip_lease_free(tgohip_lease* l) {
  if (!l) return;
  l->l->release();
  delete l->l;
  delete l;
}
