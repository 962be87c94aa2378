// hostlogic.h -- host-side mirrors of tgo's prefix block pool
// (internal/prefix/prefix.go, lease.go, hash.go).
#pragma once
#include <stdint.h>
#include <string.h>

#include <map>
#include <string>
#include <vector>

struct Hash32 {
  uint8_t b[32];
  Hash32() { memset(b, 0, 32); }
  bool operator<(const Hash32& o) const { return memcmp(b, o.b, 32) < 0; }
  bool operator==(const Hash32& o) const { return memcmp(b, o.b, 32) == 0; }
};

Hash32 prefix_seed(int scope, const std::string& domain, const std::string& salt);
Hash32 prefix_chain(const Hash32& prev, const int32_t* ids, int n);

struct PrefixStats {
  int64_t acquires = 0, hits = 0, reused = 0, prompt = 0, evictions = 0, publishes = 0,
          adoptions = 0, in_use = 0, cached = 0, free = 0;
};

struct PrefixLease;

// prefix.Pool: block bookkeeping, refcounts, an intrusive LRU of cached
// blocks (refcount 0 with a hash entry) and the hash -> block map.
struct PrefixPool {
  struct Blk {
    Hash32 hash;
    bool published = false;
    int refs = 0;
    int prev = -1, next = -1;
  };
  int block, blocks, scope;  // scope: 0 process, 1 session, 2 off
  std::vector<Blk> blk;
  std::map<Hash32, int> entry;
  std::vector<int> free;
  int head, tail;
  PrefixStats st;

  PrefixPool(int block, int blocks, int scope);
  int acquire(const int32_t* ids, int n, const std::string& session, const std::string& salt,
              int reserve, PrefixLease** out);
  int alloc(int n, std::vector<int>& out);
  bool take(int& out);
  void evict(int id);
  void hold(int id);
  void drop(int id);
  void release_taken(int id);
  void lru_push(int id);
  void lru_remove(int id);
};

// prefix.Lease: one sequence's hold on the blocks its KV lives in.
struct PrefixLease {
  PrefixPool* pool = nullptr;
  Hash32 seed;
  std::vector<int32_t> ids;
  std::vector<int> blocks;
  std::vector<Hash32> hashes;
  int matched = 0, reused = 0, published = 0;
  bool released = false;

  int grow(int n);
  int commit(const int32_t* ids, int n);
  void publish(int written);
  void release();
};
