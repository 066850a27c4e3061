// tk_added.hip -- added-token literal extraction ahead of the pretokenizer.
//
// Hugging Face tokenizers 0.22.2 splits a text at its added-token literals
// before anything else runs: the leftmost match wins, the longest one at
// that position, and the scan goes on after it (an Aho-Corasick search in
// leftmost-longest mode); each literal becomes its own id and the text
// between literals is normalized, pretokenized and merged segment by
// segment. The reference does the split on the host and routes every input
// that holds a literal to its CPU engine (src/toktier/frontend/added.py:
// 503-533, crates/toktier-routing-core/src/runtime.rs:527-536, :641-662).
// Here the split runs on the device, in one kernel ahead of k_pretok, and
// the segments stay on the GPU path as documents of their own.
//
// Which literals are chosen is a function of the text alone, so every
// block decides it for its own bytes without waiting for another:
//   - a candidate is a position where some literal matches; its literal is
//     the longest one matching there (a walk down the trie of the
//     literals);
//   - a candidate that no earlier candidate reaches (every candidate in the
//     lmax - 1 bytes before it ends at or before it) is certain: it is
//     chosen whatever was chosen before it;
//   - any other candidate is decided by going back to the nearest certain
//     candidate and scanning forward from there, choosing each candidate
//     that starts at or after the end of the last choice.
// A block stages its 4096 bytes with AD_BACK bytes before and AD_AHEAD
// after (and the trie's edge table, when it fits) in LDS, finds the
// candidates of the
// staged range, decides every candidate whose literal can reach its bytes,
// and writes its own 64 mask words whole: document starts at each chosen
// literal's first byte and just past its end, the first byte in lits, the
// others in litb; the literal's id goes to tok at its first byte. Chains of
// overlapping candidates longer than the staged range are followed in HBM
// (the text does not change), which is slow but only arises in texts built
// to overlap literals. k_pretok then forms no piece on a literal's bytes.
#include "tk_device.h"

#include <hip/hip_ext.h>

namespace tk {

namespace {

constexpr int AD_BACK = 512;    // > 2 * ADDED_MAX_LEN: a reaching literal
                                // and its certainty window are staged
constexpr int AD_AHEAD = 256;   // > ADDED_MAX_LEN: a walk from the block's
                                // last byte stays staged
constexpr int AD_STAGE = AD_BACK + ADDED_BLOCK_BYTES + AD_AHEAD;
constexpr int AD_CAND = AD_BACK + ADDED_BLOCK_BYTES;  // candidates staged
constexpr int AD_LIST = 1024;   // listed first-byte positions per block
static_assert(AD_STAGE % 16 == 0, "16-byte staging");
static_assert(2 * ADDED_MAX_LEN < AD_BACK && ADDED_MAX_LEN < AD_AHEAD,
              "staged margins hold a literal and its certainty window");

__device__ __forceinline__ bool gate_hit(const DevAdded& a, uint32_t b) {
  const uint64_t g = b < 64 ? a.gate[0] : b < 128 ? a.gate[1]
                   : b < 192 ? a.gate[2] : a.gate[3];
  return (g >> (b & 63)) & 1;
}

// the trie edge (node, byte), or ~0 when there is none
__device__ __forceinline__ uint64_t edge_find(const uint64_t* tab,
                                              uint32_t size, uint32_t key) {
  uint32_t i = added_slot(key, size);
  for (;;) {
    const uint64_t e = tab[i];
    if ((uint32_t)(e >> 36) == key) return e;
    if (e == ~0ULL) return ~0ULL;
    i = i + 1 == size ? 0 : i + 1;
  }
}

// The trie walk from p: len << 16 | (literal + 1) for the longest literal
// that matches there, 0 for none. It stops at the text end and at the next
// document start (a literal never spans two documents). bytes[q - base] is
// the byte at q, dmw[(q >> 6) - dm_base] its document-start word (dmw may
// be null), tab the edge table (LDS or HBM).
__device__ uint32_t trie_match(const DevAdded& a, const uint8_t* bytes,
                               int64_t base, int64_t nb, const uint64_t* dmw,
                               int64_t dm_base, const uint64_t* tab,
                               int64_t p) {
  if (!gate_hit(a, bytes[p - base])) return 0;
  uint32_t v = 0, best = 0;
  for (uint32_t j = 0; j < a.lmax; ++j) {
    const int64_t q = p + j;
    if (q >= nb) break;
    if (j > 0 && dmw && ((dmw[(q >> 6) - dm_base] >> (q & 63)) & 1)) break;
    const uint64_t e = edge_find(tab, a.tab_size, (v << 8) | bytes[q - base]);
    if (e == ~0ULL) break;
    v = (uint32_t)(e >> 16) & 0xFFFFF;
    if (e & 0xFFFF) best = ((j + 1) << 16) | (uint32_t)(e & 0xFFFF);
  }
  return best;
}

// L: the edge table and the literal lengths are read from the block's LDS
// copies (one code path per case, so no pointer mixes LDS and HBM: such a
// pointer makes flat loads, which wait for every memory operation in
// flight).
template <bool L>
struct Block {
  const DevAdded& a;
  const uint8_t* text;
  int64_t nb;
  const uint64_t* dm;       // document starts (batch) or nullptr
  const uint16_t* scand;    // staged candidates [s0, s0 + AD_CAND): lit + 1
  const uint8_t* slen;      // literal lengths (LDS copy when L)
  int64_t s0;

  // literal + 1 of the candidate at q, 0 for none
  __device__ __forceinline__ uint32_t cand(int64_t q) const {
    if (q < 0) return 0;
    const int64_t j = q - s0;
    if ((uint64_t)j < (uint64_t)AD_CAND) return scand[j];
    return q < nb ? trie_match(a, text, 0, nb, dm, 0, a.tab, q) & 0xFFFF : 0;
  }
  __device__ __forceinline__ int64_t len(uint32_t c) const {
    return L ? slen[c - 1] : a.len[c - 1];
  }
  // no candidate in [q - lmax + 1, q) reaches past q
  __device__ bool certain(int64_t q) const {
    for (int64_t j = q - 1; j > q - (int64_t)a.lmax && j >= 0; --j) {
      const uint32_t c = cand(j);
      if (c && j + len(c) > q) return false;
    }
    return true;
  }
  // is candidate p chosen?
  __device__ bool chosen(int64_t p) const {
    if (certain(p)) return true;
    // p is reached by an earlier candidate, so each step back finds one
    // within lmax - 1 bytes, until a certain one
    int64_t h = p;
    for (;;) {
      int64_t j = h - 1;
      while (j >= 0 && !cand(j)) --j;
      if (j < 0) return true;  // (cannot happen: h is reached by one)
      h = j;
      if (certain(h)) break;
    }
    int64_t cover = h + len(cand(h));
    for (int64_t q = h + 1; q < p; ++q) {
      const uint32_t c = cand(q);
      if (c && q >= cover) cover = q + len(c);
    }
    return p >= cover;
  }
};

__device__ __forceinline__ void set_bits(unsigned long long* words, int64_t from,
                                         int64_t lo, int64_t hi) {
  // bits [lo, hi) of the block whose first byte is `from` (clipped to it)
  if (lo < from) lo = from;
  if (hi > from + ADDED_BLOCK_BYTES) hi = from + ADDED_BLOCK_BYTES;
  while (lo < hi) {
    const int k = (int)((lo - from) >> 6);
    const int64_t end = from + 64 * (k + 1) < hi ? from + 64 * (k + 1) : hi;
    const int b0 = (int)((lo - from) & 63), n = (int)(end - lo);
    atomicOr(&words[k], n >= 64 ? ~0ULL : (((1ULL << n) - 1) << b0));
    lo = end;
  }
}

template <bool L>
__global__ __launch_bounds__(256) void k_added(DevAdded a, DevWork w,
                                               const uint64_t* host_dm,
                                               uint64_t* docmask,
                                               int64_t nwords) {
  __shared__ __align__(16) uint8_t sx[AD_STAGE];
  __shared__ uint64_t stab[ADDED_TAB_LDS];
  __shared__ uint16_t scand[AD_CAND];
  __shared__ uint8_t slen_l[ADDED_LEN_LDS];
  __shared__ unsigned long long sdm[64], slits[64], slitb[64];
  __shared__ uint64_t shdm[AD_STAGE / 64];  // caller's document starts
  __shared__ uint32_t scount;
  __shared__ uint16_t slist[AD_LIST];  // staged positions of first bytes
  __shared__ uint32_t slist_n;
  const int tid = threadIdx.x;
  const int64_t B = (int64_t)blockIdx.x * ADDED_BLOCK_BYTES;
  const int64_t s0 = B - AD_BACK, nb = w.nb;
  int hit = 0;
  // (the staging's 16-byte loads all issued before any is used)
  constexpr int SPT = (AD_STAGE / 16 + 255) / 256;
  uint4 sv[SPT];
#pragma unroll
  for (int i = 0; i < SPT; ++i) {
    const int j = tid + 256 * i;
    const int64_t p = s0 + 16 * j;
    sv[i] = make_uint4(0, 0, 0, 0);
    if (j < AD_STAGE / 16 && p >= 0 && p + 16 <= nb &&
        ((uintptr_t)(w.text + p) & 15) == 0)
      sv[i] = *reinterpret_cast<const uint4*>(w.text + p);
  }
#pragma unroll
  for (int i = 0; i < SPT; ++i) {
    const int j = tid + 256 * i;
    if (j >= AD_STAGE / 16) break;
    const int64_t p = s0 + 16 * j;
    uint4 v = sv[i];
    if (!(p >= 0 && p + 16 <= nb && ((uintptr_t)(w.text + p) & 15) == 0)) {
      uint32_t x[4] = {0, 0, 0, 0};
      for (int k = 0; k < 16; ++k) {
        const int64_t q = p + k;
        if (q >= 0 && q < nb) x[k >> 2] |= (uint32_t)w.text[q] << (8 * (k & 3));
      }
      v = make_uint4(x[0], x[1], x[2], x[3]);
    }
    *reinterpret_cast<uint4*>(sx + 16 * j) = v;
    // a first byte of some literal in the candidate range
    if (16 * j < AD_CAND) {
      const uint32_t x[4] = {v.x, v.y, v.z, v.w};
      for (int k = 0; k < 16; ++k) {
        const int64_t q = p + k;
        hit |= (int)gate_hit(a, (x[k >> 2] >> (8 * (k & 3))) & 0xFF) &
               (q >= 0 && q < nb);
      }
    }
  }
  if (tid < 64) sdm[tid] = slits[tid] = slitb[tid] = 0;
  if (tid == 0) scount = slist_n = 0;
  const int64_t w0 = s0 >> 6;  // s0 is a multiple of 64
  if (host_dm && tid < AD_STAGE / 64) {
    const int64_t wd = w0 + tid;
    shdm[tid] = (wd >= 0 && wd < nwords) ? host_dm[wd] : 0;
  }
  const bool any = __syncthreads_or(hit) != 0 && a.n > 0;
  if (a.newline_cuts) {
    // Laguna's stage 0: a (?:\r?\n)+ run opens a new part where it begins:
    // at a '\n', or a '\r' before a '\n', that does not continue a run
    // (a '\n', or the '\r' of '\r\n', just before it). A run never
    // reaches across a caller's document start; literals never begin or
    // end with CR or LF here (the engine refuses such tables), so the
    // raw bytes give the same runs as the text between literals.
    for (int k = 0; k < 16; ++k) {
      const int j = 16 * tid + k;          // offset in the block
      const int64_t i = B + j;
      if (i >= nb) break;
      const int x = j + AD_BACK;           // its index in sx
      const uint32_t b0 = sx[x], bn = sx[x + 1], bp = sx[x - 1];
      auto hdoc = [&](int64_t q) {
        return host_dm && ((shdm[(q >> 6) - w0] >> (q & 63)) & 1);
      };
      const bool unit = b0 == '\n' ||
          (b0 == '\r' && i + 1 < nb && bn == '\n' && !hdoc(i + 1));
      const bool cont = i > 0 && !hdoc(i) &&
          (bp == '\n' || (bp == '\r' && b0 == '\n'));
      if (unit && !cont) set_bits(sdm, B, i, i + 1);
    }
  }
  if (any) {
    if (L) {
      // every load first, then the stores (a load-store loop waits for
      // each load in turn)
      constexpr int TPT = (ADDED_TAB_LDS + 255) / 256, LPT = (ADDED_LEN_LDS + 255) / 256;
      uint64_t te[TPT];
      uint8_t le[LPT];
#pragma unroll
      for (int i = 0; i < TPT; ++i) {
        const uint32_t k = tid + 256 * i;
        te[i] = k < a.tab_size ? a.tab[k] : 0;
      }
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        const uint32_t k = tid + 256 * i;
        le[i] = k < a.n ? a.len[k] : 0;
      }
#pragma unroll
      for (int i = 0; i < TPT; ++i)
        if (tid + 256 * i < a.tab_size) stab[tid + 256 * i] = te[i];
#pragma unroll
      for (int i = 0; i < LPT; ++i)
        if (tid + 256 * i < a.n) slen_l[tid + 256 * i] = le[i];
    }
    // The staged positions that hold some literal's first byte, listed
    // (one LDS counter update per wave): the trie walks then run one
    // position per lane, instead of every lane's walk holding up its wave
    // on each of its positions in turn. More than AD_LIST of them (a text
    // of first bytes): every position is walked in place.
    for (int j = tid; j < AD_CAND; j += 256) scand[j] = 0;
    {
      const int lane = tid & 63;
      for (int j0 = tid - lane; j0 < AD_CAND; j0 += 256) {
        const int j = j0 + lane;
        const int64_t p = s0 + j;
        const bool g = j < AD_CAND && p >= 0 && p < nb && gate_hit(a, sx[j]);
        const uint64_t bm = __ballot(g);
        if (!bm) continue;  // wave-uniform
        uint32_t at = 0;
        if (lane == 0) at = atomicAdd(&slist_n, (uint32_t)__popcll(bm));
        at = __shfl(at, 0) + (uint32_t)__popcll(bm & ((1ULL << lane) - 1));
        if (g && at < AD_LIST) slist[at] = (uint16_t)j;
      }
    }
    __syncthreads();
    const uint32_t nlist = slist_n;
    const bool listed = nlist <= AD_LIST;
    auto match = [&](int j) {
      const int64_t p = s0 + j;
      uint16_t c = 0;
      if (p >= 0 && p < nb) {
        if (host_dm)
          c = (uint16_t)trie_match(a, sx, s0, nb, shdm, w0, L ? stab : a.tab, p);
        else
          c = (uint16_t)trie_match(a, sx, s0, nb, nullptr, 0, L ? stab : a.tab, p);
      }
      scand[j] = c;
    };
    if (listed) {
      for (uint32_t k = tid; k < nlist; k += 256) match(slist[k]);
    } else {
      for (int j = tid; j < AD_CAND; j += 256) match(j);
    }
    __syncthreads();
    const Block<L> blk{a, w.text, nb, host_dm, scand, slen_l, s0};
    // every candidate whose literal, or the document start just past it,
    // falls on the block's bytes (candidates are listed positions, when
    // listed)
    uint32_t mine = 0;
    const uint32_t nj = listed ? nlist : (uint32_t)AD_CAND;
    for (uint32_t k = tid; k < nj; k += 256) {
      const int j = listed ? (int)slist[k] : (int)k;
      if (j < AD_BACK - ADDED_MAX_LEN) continue;
      const uint32_t c = scand[j];
      if (!c) continue;
      const int64_t s = s0 + j, e = s + blk.len(c);
      if (e < B || !blk.chosen(s)) continue;
      set_bits(sdm, B, s, s + 1);
      if (e < nb) set_bits(sdm, B, e, e + 1);
      set_bits(slits, B, s, s + 1);
      set_bits(slitb, B, s + 1, e);
      if (s >= B) {
        w.tok[s] = a.id[c - 1];
        for (int64_t q = s + 1; q < e; ++q) w.tok[q] = INVALID_ID;
        ++mine;
      }
    }
    if (mine) atomicAdd(&scount, mine);
  }
  __syncthreads();
  if (tid < 64) {
    const int64_t wd = (B >> 6) + tid;
    if (wd < nwords) {
      docmask[wd] = (host_dm ? host_dm[wd] : 0ULL) | sdm[tid];
      w.lits[wd] = slits[tid];
      w.litb[wd] = slitb[tid];
    }
  }
  if (tid == 0 && scount) atomicAdd(w.nlit, scount);
}

}  // namespace

hipError_t launch_added(const DevAdded& a, const DevWork& w,
                        const uint64_t* host_dm, hipStream_t s,
                        hipEvent_t start, hipEvent_t stop) {
  // the words k_pretok reads; the caller's mask holds nb / 64 + 2 of them
  const int64_t nwords = (w.nb + 63) / 64 + 2;
  uint64_t* dm = const_cast<uint64_t*>(w.docmask);
  const uint32_t g = (uint32_t)((nwords * 64 + ADDED_BLOCK_BYTES - 1) / ADDED_BLOCK_BYTES);
  const bool lds = a.tab_size <= (uint32_t)ADDED_TAB_LDS &&
                   a.n <= (uint32_t)ADDED_LEN_LDS;
  auto k = lds ? k_added<true> : k_added<false>;
  if (start || stop)
    hipExtLaunchKernelGGL(k, dim3(g), dim3(256), 0, s, start, stop, 0,
                          a, w, host_dm, dm, nwords);
  else
    hipLaunchKernelGGL(k, dim3(g), dim3(256), 0, s, a, w, host_dm, dm, nwords);
  return hipGetLastError();
}

}  // namespace tk
