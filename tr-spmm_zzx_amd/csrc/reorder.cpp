// TCA row reorder (trs_tca_reorder in include/trspmm.h): rows with similar column sets are
// clustered so that they land in the same 16-row windows, which raises the dense-tile share of the
// format and the reuse of gathered B rows.  Same procedure as the reference's
// spmm/tr_csr_fp16/tr_tca_reorder.py:44-357, native and deterministic:
//
//   level 1  sets = the rows' column lists.  Candidate pairs from MinHash LSH (b bands of r
//            signature values, (b, r) minimising the equally weighted false-positive and
//            false-negative areas for the Jaccard threshold, as the reference's LSH library
//            does), scored by exact Jaccard, merged greedily in order of similarity by a
//            union-find whose clusters close once they reach `thres` rows (:145-210)
//   level 2  sets = the column unions of the level-1 clusters, same procedure, clusters close at
//            `cluster_thres` level-1 clusters (:212-323)
//   order    level-2 groups in order of their first cluster, level-1 clusters inside a group in
//            index order, rows of a cluster in ascending order (:325-340)
//
// MinHash family (params.minhash): 1 (default) = the reference's LSH library (datasketch, whose
// MinHash and MinHashLSH the reference calls at :84-90, :121-123, :226-249): element e hashes to
// the first 4 bytes (little-endian) of SHA-1 of its decimal string, permutation k maps it to
// ((a_k e + b_k) mod 2^64) mod (2^61 - 1), low 32 bits, with (a_k, b_k) the k-th pair of draws
// a in [1, 2^61 - 1), b in [0, 2^61 - 1) of numpy's legacy RandomState(seed) -- seed 1 is the
// library's default -- and a band matches when its r values are equal; 0 = a 64-bit mixing hash
// (faster, other candidates).
// Deviations (forced by scale or by the reference being non-deterministic):
//   * an LSH bucket with more than `bucket_span` + 1 sets pairs each set with the next
//     `bucket_span` sets of the bucket only (the reference pairs all, O(bucket^2));
//     bucket_span <= 0 pairs all, as the reference;
//   * equal similarities pop in (pair key) order; the reference's queue order for ties depends on
//     Python's per-process string hashing.
// Extension (align_window = W > 0, no reference counterpart): level-1 merges that would exceed W
// rows are skipped, and the clusters are packed into whole W-row windows (aligned_order), so a
// cluster never straddles two windows.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <queue>
#include <string>
#include <vector>

#include <omp.h>

#include "format.hpp"

namespace {

// Sets in CSR form: elements of set i are e[off[i] .. off[i+1]), sorted, unique.
struct Sets {
  std::vector<int64_t> off;
  std::vector<int32_t> e;
  int32_t size() const { return (int32_t)off.size() - 1; }
  int64_t len(int32_t i) const { return off[i + 1] - off[i]; }
};

uint64_t mix64(uint64_t x) {   // splitmix64 finaliser
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

// ---- the reference LSH library's MinHash family --------------------------------------------------
uint32_t rotl32(uint32_t x, int k) { return (x << k) | (x >> (32 - k)); }

// SHA-1 (FIPS 180-4) of a message of fewer than 56 bytes (one block); returns digest bytes 0..3 read
// little-endian.
uint32_t sha1_first32(const unsigned char* msg, size_t len) {
  unsigned char block[64] = {0};
  std::memcpy(block, msg, len);
  block[len] = 0x80;
  const uint64_t bits = (uint64_t)len * 8;
  for (int i = 0; i < 8; ++i) block[63 - i] = (unsigned char)(bits >> (8 * i));
  uint32_t w[80];
  for (int i = 0; i < 16; ++i)
    w[i] = (uint32_t)block[4 * i] << 24 | (uint32_t)block[4 * i + 1] << 16 | (uint32_t)block[4 * i + 2] << 8 |
           (uint32_t)block[4 * i + 3];
  for (int i = 16; i < 80; ++i) w[i] = rotl32(w[i - 3] ^ w[i - 8] ^ w[i - 14] ^ w[i - 16], 1);
  uint32_t a = 0x67452301u, b = 0xEFCDAB89u, c = 0x98BADCFEu, d = 0x10325476u, e = 0xC3D2E1F0u;
  for (int i = 0; i < 80; ++i) {
    uint32_t f, k;
    if (i < 20) { f = (b & c) | (~b & d); k = 0x5A827999u; }
    else if (i < 40) { f = b ^ c ^ d; k = 0x6ED9EBA1u; }
    else if (i < 60) { f = (b & c) | (b & d) | (c & d); k = 0x8F1BBCDCu; }
    else { f = b ^ c ^ d; k = 0xCA62C1D6u; }
    const uint32_t t = rotl32(a, 5) + f + e + k + w[i];
    e = d; d = c; c = rotl32(b, 30); b = a; a = t;
  }
  const uint32_t h0 = 0x67452301u + a;   // digest bytes 0..3, big-endian
  return (h0 >> 24) | ((h0 >> 8) & 0xff00u) | ((h0 << 8) & 0xff0000u) | (h0 << 24);
}

// Mersenne Twister MT19937 with numpy's legacy RandomState seeding of an integer seed and its
// bounded 64-bit draws (mask the range, reject values past it; two 32-bit outputs per 64-bit one,
// the first the high half).
class Mt19937 {
 public:
  explicit Mt19937(uint32_t seed) {
    mt_[0] = seed;
    for (int i = 1; i < 624; ++i) mt_[i] = 1812433253u * (mt_[i - 1] ^ (mt_[i - 1] >> 30)) + (uint32_t)i;
  }
  uint32_t next32() {
    if (pos_ >= 624) {
      for (int i = 0; i < 624; ++i) {
        const uint32_t y = (mt_[i] & 0x80000000u) | (mt_[(i + 1) % 624] & 0x7fffffffu);
        mt_[i] = mt_[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
      }
      pos_ = 0;
    }
    uint32_t y = mt_[pos_++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
  }
  // uniform in [low, high)
  uint64_t bounded(uint64_t low, uint64_t high) {
    const uint64_t rng = high - low - 1;
    if (rng == 0) return low;
    uint64_t mask = rng;
    for (int s = 1; s < 64; s <<= 1) mask |= mask >> s;
    uint64_t v;
    if (rng <= 0xffffffffull) {
      do v = next32() & mask; while (v > rng);
    } else {
      do {
        const uint64_t hi = next32();
        v = ((hi << 32) | next32()) & mask;
      } while (v > rng);
    }
    return low + v;
  }

 private:
  uint32_t mt_[624];
  int pos_ = 624;
};

constexpr uint64_t kMersenne61 = (1ull << 61) - 1;
uint64_t mod_mersenne61(uint64_t x) {
  uint64_t r = (x & kMersenne61) + (x >> 61);
  return r >= kMersenne61 ? r - kMersenne61 : r;
}

// The first `used` permutations (a_k, b_k) of seed.
void reference_permutations(uint64_t seed, int used, std::vector<uint64_t>& a, std::vector<uint64_t>& b) {
  Mt19937 g((uint32_t)seed);
  a.resize(used);
  b.resize(used);
  for (int k = 0; k < used; ++k) {
    a[k] = g.bounded(1, kMersenne61);
    b[k] = g.bounded(0, kMersenne61);
  }
}

double jaccard(const Sets& S, int32_t a, int32_t b) {
  const int32_t *x = S.e.data() + S.off[a], *xe = S.e.data() + S.off[a + 1];
  const int32_t *y = S.e.data() + S.off[b], *ye = S.e.data() + S.off[b + 1];
  const int64_t na = xe - x, nb = ye - y;
  if (na == 0 || nb == 0) return 0.0;
  int64_t inter = 0;
  while (x < xe && y < ye) {
    if (*x < *y) ++x;
    else if (*y < *x) ++y;
    else { ++inter; ++x; ++y; }
  }
  const int64_t uni = na + nb - inter;
  return uni > 0 ? (double)inter / (double)uni : 0.0;
}

// Area of the LSH false-positive / false-negative probability over [lo, hi] (Simpson, fine grid).
double area(double lo, double hi, int b, int r, bool positive) {
  const int n = 2000;
  const double h = (hi - lo) / n;
  auto f = [&](double s) {
    const double p = 1.0 - std::pow(1.0 - std::pow(s, r), b);   // P(candidate | similarity s)
    return positive ? p : 1.0 - p;
  };
  double acc = f(lo) + f(hi);
  for (int i = 1; i < n; ++i) acc += f(lo + i * h) * (i % 2 ? 4.0 : 2.0);
  return acc * h / 3.0;
}

void lsh_bands(double t, int num_perm, int& bands, int& rows) {
  double best = 1e300;
  bands = 1;
  rows = 1;
  for (int b = 1; b <= num_perm; ++b)
    for (int r = 1; r <= num_perm / b; ++r) {
      const double err = 0.5 * area(0.0, t, b, r, true) + 0.5 * area(t, 1.0, b, r, false);
      if (err < best) { best = err; bands = b; rows = r; }
    }
}

struct Pair {
  double sim;
  int32_t p1, p2;   // orientation matters: equal-size merges fold p2 into p1
};
uint64_t pair_key(int32_t a, int32_t b, int64_t n) {
  return a < b ? (uint64_t)a * (uint64_t)n + (uint64_t)b : (uint64_t)b * (uint64_t)n + (uint64_t)a;
}

// Open-addressing set of pair keys (the reference's `sset`), with tombstones.
class KeySet {
 public:
  explicit KeySet(size_t expect) {
    size_t cap = 1024;
    while (cap < expect * 2 + 16) cap <<= 1;
    slot_.assign(cap, kEmpty);
  }
  bool contains(uint64_t k) const {
    for (size_t i = hash(k);; i = (i + 1) & (slot_.size() - 1)) {
      if (slot_[i] == k) return true;
      if (slot_[i] == kEmpty) return false;
    }
  }
  void insert(uint64_t k) {
    if ((used_ + 1) * 2 > slot_.size()) grow();
    size_t tomb = SIZE_MAX;
    for (size_t i = hash(k);; i = (i + 1) & (slot_.size() - 1)) {
      if (slot_[i] == k) return;
      if (slot_[i] == kTomb && tomb == SIZE_MAX) tomb = i;
      if (slot_[i] == kEmpty) {
        if (tomb != SIZE_MAX) slot_[tomb] = k;
        else { slot_[i] = k; ++used_; }
        return;
      }
    }
  }
  void erase(uint64_t k) {
    for (size_t i = hash(k);; i = (i + 1) & (slot_.size() - 1)) {
      if (slot_[i] == k) { slot_[i] = kTomb; return; }
      if (slot_[i] == kEmpty) return;
    }
  }

 private:
  static constexpr uint64_t kEmpty = ~0ull, kTomb = ~0ull - 1;
  size_t hash(uint64_t k) const { return (size_t)mix64(k) & (slot_.size() - 1); }
  void grow() {
    std::vector<uint64_t> old;
    old.swap(slot_);
    slot_.assign(old.size() * 2, kEmpty);
    used_ = 0;
    for (uint64_t k : old)
      if (k != kEmpty && k != kTomb) insert(k);
  }
  std::vector<uint64_t> slot_;
  size_t used_ = 0;
};

// MinHash signatures: sig[i * used + k] = the minimum over set i's elements of hash k (empty sets
// keep 0xffffffff), in the family params.minhash selects.
std::vector<uint32_t> signatures(const Sets& S, const trs_reorder_params& prm, int used) {
  const int32_t n = S.size();
  std::vector<uint32_t> sig((size_t)n * used, 0xffffffffu);
  if (prm.minhash == 1) {
    std::vector<uint64_t> pa, pb;
    reference_permutations(prm.seed, used, pa, pb);
    // element hashes, once per distinct element: a table over [0, max] when that is not much
    // larger than the element count (columns of a matrix), else over the sorted distinct values
    auto sha = [](int64_t v) {
      char buf[24];
      const int len = std::snprintf(buf, sizeof buf, "%lld", (long long)v);
      return sha1_first32(reinterpret_cast<const unsigned char*>(buf), (size_t)len);
    };
    int64_t top = -1;
    for (int32_t v : S.e) top = std::max<int64_t>(top, v);
    const bool dense = top + 1 <= std::max<int64_t>((int64_t)S.e.size() * 4, 1 << 20);
    std::vector<int32_t> distinct;
    if (!dense) {
      distinct = S.e;
      std::sort(distinct.begin(), distinct.end());
      distinct.erase(std::unique(distinct.begin(), distinct.end()), distinct.end());
    }
    const int64_t nh = dense ? top + 1 : (int64_t)distinct.size();
    std::vector<uint32_t> hv((size_t)nh);
#pragma omp parallel for schedule(static, 4096)
    for (int64_t v = 0; v < nh; ++v) hv[v] = sha(dense ? v : distinct[v]);
    auto hash_of = [&](int32_t e) -> uint64_t {
      if (dense) return hv[e];
      return hv[std::lower_bound(distinct.begin(), distinct.end(), e) - distinct.begin()];
    };
#pragma omp parallel for schedule(dynamic, 256)
    for (int32_t i = 0; i < n; ++i) {
      uint32_t* s = sig.data() + (size_t)i * used;
      for (int64_t j = S.off[i]; j < S.off[i + 1]; ++j) {
        const uint64_t h = hash_of(S.e[j]);
        for (int k = 0; k < used; ++k) {
          const uint32_t v = (uint32_t)(mod_mersenne61(pa[k] * h + pb[k]) & 0xffffffffu);
          if (v < s[k]) s[k] = v;
        }
      }
    }
    return sig;
  }
  std::vector<uint64_t> coef(used);
  for (int k = 0; k < used; ++k) coef[k] = mix64(prm.seed * 0x2545f4914f6cdd1dull + (uint64_t)k + 1);
#pragma omp parallel for schedule(dynamic, 256)
  for (int32_t i = 0; i < n; ++i) {
    uint32_t* s = sig.data() + (size_t)i * used;
    for (int64_t j = S.off[i]; j < S.off[i + 1]; ++j) {
      const uint64_t base = mix64((uint64_t)(uint32_t)S.e[j]);
      for (int k = 0; k < used; ++k) {
        const uint32_t h = (uint32_t)(mix64(base ^ coef[k]) >> 32);
        if (h < s[k]) s[k] = h;
      }
    }
  }
  return sig;
}

// Candidate pairs (a < b) of non-empty sets: MinHash LSH, or every pair when exhaustive.
std::vector<std::pair<int32_t, int32_t>> candidates(const Sets& S, const trs_reorder_params& prm) {
  const int32_t n = S.size();
  std::vector<std::pair<int32_t, int32_t>> out;
  if (prm.exhaustive) {
    for (int32_t a = 0; a < n; ++a)
      if (S.len(a))
        for (int32_t b = a + 1; b < n; ++b)
          if (S.len(b)) out.push_back({a, b});
    return out;
  }
  int bands, r;
  lsh_bands(prm.lsh_threshold, prm.num_perm, bands, r);
  const int used = bands * r;
  const std::vector<uint32_t> sig = signatures(S, prm, used);
  // per band: sets sorted by their band values; runs of equal values are buckets
  std::vector<std::vector<std::pair<int32_t, int32_t>>> per_band(bands);
  const size_t span = prm.bucket_span > 0 ? (size_t)prm.bucket_span : SIZE_MAX;
#pragma omp parallel for schedule(dynamic, 1)
  for (int t = 0; t < bands; ++t) {
    const uint32_t* base = sig.data() + (size_t)t * r;
    auto band = [&](int32_t i) { return base + (size_t)i * used; };
    auto less = [&](int32_t x, int32_t y) {
      const uint32_t *a = band(x), *b = band(y);
      for (int k = 0; k < r; ++k)
        if (a[k] != b[k]) return a[k] < b[k];
      return x < y;
    };
    auto same = [&](int32_t x, int32_t y) { return std::equal(band(x), band(x) + r, band(y)); };
    std::vector<int32_t> ids;
    ids.reserve(n);
    for (int32_t i = 0; i < n; ++i)
      if (S.len(i)) ids.push_back(i);
    std::sort(ids.begin(), ids.end(), less);
    auto& dst = per_band[t];
    for (size_t a = 0; a < ids.size();) {
      size_t e = a;
      while (e < ids.size() && same(ids[e], ids[a])) ++e;
      for (size_t x = a; x < e; ++x)
        for (size_t y = x + 1; y < e && y - x <= span; ++y) dst.push_back({ids[x], ids[y]});
      a = e;
    }
  }
  size_t total = 0;
  for (auto& v : per_band) total += v.size();
  std::vector<uint64_t> keys;
  keys.reserve(total);
  for (auto& v : per_band) {
    for (auto& p : v) keys.push_back(pair_key(p.first, p.second, n));
    std::vector<std::pair<int32_t, int32_t>>().swap(v);
  }
  std::sort(keys.begin(), keys.end());
  keys.erase(std::unique(keys.begin(), keys.end()), keys.end());
  out.resize(keys.size());
  for (size_t i = 0; i < keys.size(); ++i) out[i] = {(int32_t)(keys[i] / (uint64_t)n), (int32_t)(keys[i] % (uint64_t)n)};
  return out;
}

// Greedy union-find clustering of the sets (tr_tca_reorder.py:145-210 / :282-323); returns the
// root of every set.  capped: a merge that would exceed `thres` members is skipped (window-aligned
// mode) instead of performed and closed.
std::vector<int32_t> cluster(const Sets& S, int32_t thres, const trs_reorder_params& prm, bool capped = false) {
  const int32_t n = S.size();
  const auto cand = candidates(S, prm);
  std::vector<Pair> init(cand.size());
#pragma omp parallel for schedule(dynamic, 4096)
  for (int64_t i = 0; i < (int64_t)cand.size(); ++i)
    init[i] = {jaccard(S, cand[i].first, cand[i].second), cand[i].first, cand[i].second};
  // max similarity first; ties by pair key, then orientation
  auto later = [n](const Pair& x, const Pair& y) {
    if (x.sim != y.sim) return x.sim < y.sim;
    const uint64_t kx = pair_key(x.p1, x.p2, n), ky = pair_key(y.p1, y.p2, n);
    if (kx != ky) return kx > ky;
    return x.p1 > y.p1;
  };
  KeySet queued(init.size());
  for (const auto& p : init) queued.insert(pair_key(p.p1, p.p2, n));
  std::priority_queue<Pair, std::vector<Pair>, decltype(later)> pq(later, std::move(init));

  std::vector<int32_t> id(n), sz(n, 1);
  std::vector<uint8_t> closed(n, 0);
  for (int32_t i = 0; i < n; ++i) id[i] = i;
  auto root = [&](int32_t i) {
    while (i != id[i]) {
      id[i] = id[id[i]];
      i = id[i];
    }
    return i;
  };
  int64_t open_clusters = n;
  while (!pq.empty() && open_clusters > 0) {
    const Pair it = pq.top();
    pq.pop();
    queued.erase(pair_key(it.p1, it.p2, n));
    const int32_t p1 = it.p1, p2 = it.p2;
    if (p1 == id[p1] && p2 == id[p2]) {
      if (closed[p1] || closed[p2]) continue;
      if (capped && sz[p1] + sz[p2] > thres) continue;
      int32_t into = p1, from = p2;
      if (sz[p1] < sz[p2]) { into = p2; from = p1; }
      id[from] = into;
      --open_clusters;
      sz[into] += sz[from];
      if (sz[into] >= thres) {
        closed[into] = 1;
        --open_clusters;
      }
    } else {
      const int32_t r1 = root(p1), r2 = root(p2);
      if (closed[r1] || closed[r2]) continue;
      const uint64_t k = pair_key(r1, r2, n);
      if (r1 != r2 && !queued.contains(k)) {
        pq.push({jaccard(S, r1, r2), r1, r2});
        queued.insert(k);
      }
    }
  }
  std::vector<int32_t> out(n);
  for (int32_t i = 0; i < n; ++i) out[i] = root(i);
  return out;
}

// Window-aligned layout: within each level-2 group, clusters (each <= W rows) are packed first-fit
// decreasing into bins of W rows; full bins are laid out in group order, the clusters of partial
// bins are packed again at the end (full bins first), so only the tail windows mix leftovers.
std::vector<int32_t> aligned_order(const std::vector<std::vector<int32_t>>& clusters,
                                   const std::vector<std::vector<int32_t>>& super, int32_t W) {
  std::vector<int32_t> order;
  auto pack = [&](const std::vector<int32_t>& ids, std::vector<std::vector<int32_t>>& bins, std::vector<int32_t>& fill) {
    std::vector<int32_t> s(ids);
    std::stable_sort(s.begin(), s.end(), [&](int32_t a, int32_t b) { return clusters[a].size() > clusters[b].size(); });
    for (int32_t c : s) {
      const int32_t sz = (int32_t)clusters[c].size();
      size_t b = 0;
      while (b < bins.size() && fill[b] + sz > W) ++b;
      if (b == bins.size()) { bins.emplace_back(); fill.push_back(0); }
      bins[b].push_back(c);
      fill[b] += sz;
    }
  };
  auto emit = [&](const std::vector<int32_t>& bin) {
    for (int32_t c : bin) order.insert(order.end(), clusters[c].begin(), clusters[c].end());
  };
  std::vector<int32_t> leftover;
  for (const auto& grp : super) {
    std::vector<std::vector<int32_t>> bins;
    std::vector<int32_t> fill;
    pack(grp, bins, fill);
    for (size_t b = 0; b < bins.size(); ++b) {
      if (fill[b] == W) emit(bins[b]);
      else leftover.insert(leftover.end(), bins[b].begin(), bins[b].end());
    }
  }
  std::vector<std::vector<int32_t>> bins;
  std::vector<int32_t> fill;
  pack(leftover, bins, fill);
  for (size_t b = 0; b < bins.size(); ++b)
    if (fill[b] == W) emit(bins[b]);
  for (size_t b = 0; b < bins.size(); ++b)
    if (fill[b] != W) emit(bins[b]);
  return order;
}

// Groups of a root array in first-appearance order, members ascending.
std::vector<std::vector<int32_t>> groups_of(const std::vector<int32_t>& roots) {
  const int32_t n = (int32_t)roots.size();
  std::vector<int32_t> gid(n, -1);
  std::vector<std::vector<int32_t>> g;
  for (int32_t i = 0; i < n; ++i) {
    const int32_t r = roots[i];
    if (gid[r] < 0) {
      gid[r] = (int32_t)g.size();
      g.emplace_back();
    }
    g[gid[r]].push_back(i);
  }
  return g;
}

}  // namespace

extern "C" void trs_reorder_params_default(trs_reorder_params* p);

namespace {
// The caller's parameters, or the defaults for NULL.  A struct_size other than this library's
// means the caller was compiled against another trspmm.h: only that first field is read.
bool take_params(const trs_reorder_params* params, trs_reorder_params& prm, const char* where) {
  trs_reorder_params_default(&prm);
  if (!params) return true;
  if (params->struct_size != (int32_t)sizeof(trs_reorder_params)) {
    trs::set_error(std::string(where) + ": trs_reorder_params.struct_size is " + std::to_string(params->struct_size) +
                   ", this library's is " + std::to_string(sizeof(trs_reorder_params)) +
                   " (initialise the parameters with trs_reorder_params_default of the same trspmm.h)");
    return false;
  }
  prm = *params;
  return true;
}
}  // namespace

extern "C" {

void trs_reorder_params_default(trs_reorder_params* p) {
  if (!p) return;
  p->struct_size = (int32_t)sizeof(trs_reorder_params);
  p->thres = 16;
  p->cluster_thres = 128;
  p->num_perm = 128;
  p->lsh_threshold = 0.2f;
  p->bucket_span = 64;
  p->num_threads = 0;
  p->exhaustive = 0;
  p->align_window = 0;
  p->seed = 1;
  p->minhash = 1;
}

int trs_lsh_bands(float threshold, int32_t num_perm, int32_t* bands, int32_t* rows) {
  if (!bands || !rows || num_perm < 1 || num_perm > 1024 || !(threshold > 0.0f && threshold < 1.0f)) {
    trs::set_error("trs_lsh_bands: num_perm in 1..1024, threshold in (0, 1), bands and rows non-NULL");
    return TRS_EINVAL;
  }
  int b = 1, r = 1;
  lsh_bands(threshold, num_perm, b, r);
  *bands = b;
  *rows = r;
  return TRS_OK;
}

int trs_minhash_signatures(const int64_t* off, const int32_t* elems, int32_t nsets, const trs_reorder_params* params,
                           int32_t count, uint32_t* sig) {
  trs_reorder_params prm;
  if (!take_params(params, prm, "trs_minhash_signatures")) return TRS_EINVAL;
  if (nsets < 0 || count < 1 || count > 1024 || !sig || (nsets > 0 && !off) || (prm.minhash != 0 && prm.minhash != 1)) {
    trs::set_error("trs_minhash_signatures: bad arguments (count in 1..1024, minhash 0 or 1)");
    return TRS_EINVAL;
  }
  Sets S;
  S.off.assign(off, off + (size_t)nsets + 1);
  if (S.off[0] != 0) {
    trs::set_error("trs_minhash_signatures: off[0] must be 0");
    return TRS_EINVAL;
  }
  for (int32_t i = 0; i < nsets; ++i)
    if (S.off[i + 1] < S.off[i]) {
      trs::set_error("trs_minhash_signatures: off must not decrease");
      return TRS_EINVAL;
    }
  if (S.off[nsets] > 0 && !elems) {
    trs::set_error("trs_minhash_signatures: NULL elements");
    return TRS_EINVAL;
  }
  S.e.assign(elems, elems + S.off[nsets]);
  for (int32_t v : S.e)
    if (v < 0) {
      trs::set_error("trs_minhash_signatures: elements must be non-negative");
      return TRS_EINVAL;
    }
  if (prm.num_threads > 0) omp_set_num_threads(prm.num_threads);
  const std::vector<uint32_t> out = signatures(S, prm, count);
  std::copy(out.begin(), out.end(), sig);
  return TRS_OK;
}

int trs_tca_reorder(const int32_t* rowptr, const int32_t* col, int32_t rows, int64_t nnz, int32_t ncols,
                    const trs_reorder_params* params, int32_t* order) {
  trs_reorder_params prm;
  if (!take_params(params, prm, "trs_tca_reorder")) return TRS_EINVAL;
  if (rows < 0 || nnz < 0 || ncols < 0 || !order || (rows > 0 && !rowptr) || (nnz > 0 && !col)) {
    trs::set_error("trs_tca_reorder: bad arguments");
    return TRS_EINVAL;
  }
  if (prm.thres < 1 || prm.cluster_thres < 1 || prm.num_perm < 1 || prm.num_perm > 1024 ||
      !(prm.lsh_threshold > 0.0f && prm.lsh_threshold < 1.0f) || prm.align_window < 0 ||
      (prm.minhash != 0 && prm.minhash != 1)) {
    trs::set_error("trs_tca_reorder: thres, cluster_thres >= 1, num_perm in 1..1024, lsh_threshold in (0, 1), "
                   "align_window >= 0, minhash 0 or 1");
    return TRS_EINVAL;
  }
  if (rows == 0) return TRS_OK;
  if (rowptr[0] != 0 || rowptr[rows] != nnz) {
    trs::set_error("trs_tca_reorder: rowptr must start at 0 and end at nnz");
    return TRS_EINVAL;
  }
  for (int32_t i = 0; i < rows; ++i)
    if (rowptr[i + 1] < rowptr[i]) {
      trs::set_error("trs_tca_reorder: rowptr not monotone");
      return TRS_EINVAL;
    }
  for (int64_t j = 0; j < nnz; ++j)
    if (col[j] < 0 || col[j] >= ncols) {
      trs::set_error("trs_tca_reorder: column index out of range");
      return TRS_ERANGE;
    }
  const int saved_threads = omp_get_max_threads();
  if (prm.num_threads > 0) omp_set_num_threads(prm.num_threads);
  try {
    // level 1: rows as sets (sorted, duplicates merged)
    Sets R;
    R.off.assign(rows + 1, 0);
    R.e.reserve(nnz);
    for (int32_t i = 0; i < rows; ++i) {
      const size_t s = R.e.size();
      R.e.insert(R.e.end(), col + rowptr[i], col + rowptr[i + 1]);
      std::sort(R.e.begin() + s, R.e.end());
      R.e.erase(std::unique(R.e.begin() + s, R.e.end()), R.e.end());
      R.off[i + 1] = (int64_t)R.e.size();
    }
    const bool aligned = prm.align_window > 0;
    const int32_t thres1 = aligned ? prm.align_window : prm.thres;
    const auto clusters = groups_of(cluster(R, thres1, prm, aligned));

    // level 2: clusters as the union of their rows' sets
    Sets C;
    C.off.assign(clusters.size() + 1, 0);
    for (size_t c = 0; c < clusters.size(); ++c) {
      const size_t s = C.e.size();
      for (int32_t row : clusters[c]) C.e.insert(C.e.end(), R.e.begin() + R.off[row], R.e.begin() + R.off[row + 1]);
      std::sort(C.e.begin() + s, C.e.end());
      C.e.erase(std::unique(C.e.begin() + s, C.e.end()), C.e.end());
      C.off[c + 1] = (int64_t)C.e.size();
    }
    const auto super = groups_of(cluster(C, prm.cluster_thres, prm));

    int32_t k = 0;
    if (aligned) {
      const auto o = aligned_order(clusters, super, prm.align_window);
      for (int32_t row : o) order[k++] = row;
    } else {
      for (const auto& grp : super)
        for (int32_t c : grp)
          for (int32_t row : clusters[c]) order[k++] = row;
    }
    if (k != rows) {
      trs::set_error("trs_tca_reorder: internal error (order is not a permutation)");
      if (prm.num_threads > 0) omp_set_num_threads(saved_threads);
      return TRS_EINVAL;
    }
  } catch (const std::bad_alloc&) {
    if (prm.num_threads > 0) omp_set_num_threads(saved_threads);
    trs::set_error("trs_tca_reorder: out of memory");
    return TRS_ENOMEM;
  }
  if (prm.num_threads > 0) omp_set_num_threads(saved_threads);
  return TRS_OK;
}

}  // extern "C"
