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
// Here the split runs on the device, in two kernels, and the segments stay
// on the GPU path as documents of their own:
//   k_added_find    per byte whose value starts a literal: walk the trie of
//                   the literals from there and keep the longest match
//                   (candidate bit + literal index); clear the masks the
//                   selection fills.
//   k_added_select  leftmost-longest choice among the candidates. A
//                   candidate that no earlier candidate reaches is always
//                   chosen: a thread starts there and walks the candidates
//                   that follow up to the next such one, choosing each one
//                   that starts at or after the end of the last choice
//                   (back-to-back literals are each their own walk). A
//                   chosen literal [s, e) marks document
//                   starts at s and e, s in lits, s+1..e-1 in litb, and
//                   writes its id at tok[s] (INVALID_ID on its other bytes).
// k_pretok then forms no piece on a literal's bytes.
#include "tk_device.h"

#include <hip/hip_ext.h>

namespace tk {

namespace {

__device__ __forceinline__ bool gate_hit(const DevAdded& a, uint32_t b) {
  const uint64_t g = b < 64 ? a.gate[0] : b < 128 ? a.gate[1]
                   : b < 192 ? a.gate[2] : a.gate[3];
  return (g >> (b & 63)) & 1;
}

__device__ __forceinline__ bool doc_start(const uint64_t* dm, int64_t i) {
  return dm && ((dm[i >> 6] >> (i & 63)) & 1);
}

// Longest literal that matches at p (its index + 1, 0 for none). The walk
// stops at the text end and, when documents are marked, at the next
// document start (a literal never spans two documents).
__device__ uint32_t longest_at(const DevAdded& a, const uint8_t* text,
                               int64_t nb, const uint64_t* dm, int64_t p) {
  uint32_t v = 0, best = 0;
  for (uint32_t j = 0; j < a.lmax; ++j) {
    const int64_t q = p + j;
    if (q >= nb || (j > 0 && doc_start(dm, q))) break;
    const uint32_t b = text[q];
    const uint2 nd = a.nodes[v];
    uint32_t child = 0;
    for (uint32_t k = 0; k < (nd.y & 0x1FF); ++k) {
      const uint32_t ed = a.edges[nd.x + k];
      if ((ed & 0xFF) == b) { child = ed >> 8; break; }
      if ((ed & 0xFF) > b) break;  // edges are sorted by byte
    }
    if (child == 0) break;  // the root is nobody's child
    v = child;
    const uint32_t term = a.nodes[v].y >> 9;
    if (term) best = term;
  }
  return best;
}

// One block per ADDED_BLOCK_BYTES bytes (64 mask words), 16 bytes per
// thread; threads 4w..4w+3 hold word w of the block.
__global__ __launch_bounds__(256) void k_added_find(DevAdded a, DevWork w,
                                                    uint64_t* docmask,
                                                    int clear_dm,
                                                    int64_t nwords) {
  const int tid = threadIdx.x;
  const int64_t p0 = (int64_t)blockIdx.x * ADDED_BLOCK_BYTES + 16 * tid;
  const int64_t nb = w.nb;
  const uint64_t* dm = clear_dm ? nullptr : docmask;
  uint8_t b[16];
  if (p0 + 16 <= nb && ((uintptr_t)(w.text + p0) & 15) == 0) {
    const uint4 v = *reinterpret_cast<const uint4*>(w.text + p0);
    const uint32_t x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 16; ++k) b[k] = (uint8_t)(x[k >> 2] >> (8 * (k & 3)));
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) b[k] = p0 + k < nb ? w.text[p0 + k] : 0;
  }
  uint32_t m16 = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int64_t p = p0 + k;
    if (p < nb && gate_hit(a, b[k])) {
      const uint32_t lit = longest_at(a, w.text, nb, dm, p);
      if (lit) {
        m16 |= 1u << k;
        w.litm[p] = lit - 1;
      }
    }
  }
  // the four 16-bit pieces of each 64-byte word
  const uint32_t m1 = __shfl_down(m16, 1), m2 = __shfl_down(m16, 2),
                 m3 = __shfl_down(m16, 3);
  if ((tid & 3) == 0) {
    const int64_t wd = p0 >> 6;
    if (wd < nwords) {
      w.cand[wd] = (uint64_t)m16 | ((uint64_t)m1 << 16) |
                   ((uint64_t)m2 << 32) | ((uint64_t)m3 << 48);
      w.lits[wd] = 0;
      w.litb[wd] = 0;
      if (clear_dm) docmask[wd] = 0;
    }
  }
}

// A candidate that no earlier candidate can cover is chosen whatever was
// chosen before it: true when every candidate j in [p - lmax + 1, p) ends
// (j + its length) at or before p.
__device__ bool certain(const DevAdded& a, const DevWork& w, int64_t p) {
  const int64_t lo = p - (int64_t)a.lmax + 1 > 0 ? p - (int64_t)a.lmax + 1 : 0;
  for (int64_t wd = lo >> 6; wd <= (p >> 6); ++wd) {
    uint64_t m = w.cand[wd];
    if (wd == (p >> 6)) m &= (1ULL << (p & 63)) - 1;      // below p
    if (wd == (lo >> 6)) m &= ~((1ULL << (lo & 63)) - 1);  // from lo
    while (m) {
      const int64_t j = wd * 64 + __builtin_ctzll(m);
      m &= m - 1;
      if (j + (int64_t)a.len[w.litm[j]] > p) return false;
    }
  }
  return true;
}

// first candidate in (p, hi), or -1
__device__ int64_t next_cand(const uint64_t* cand, int64_t p, int64_t hi,
                             int64_t nwords) {
  for (int64_t wd = (p + 1) >> 6; wd < nwords && wd * 64 < hi; ++wd) {
    uint64_t m = cand[wd];
    if (wd == ((p + 1) >> 6)) m &= ~((1ULL << ((p + 1) & 63)) - 1);
    if (m) {
      const int64_t q = wd * 64 + __builtin_ctzll(m);
      return q < hi ? q : -1;
    }
  }
  return -1;
}

__device__ void choose(const DevAdded& a, const DevWork& w, uint64_t* docmask,
                       int64_t s) {
  const uint32_t lit = w.litm[s];
  const int64_t e = s + a.len[lit];
  atomicOr((unsigned long long*)&docmask[s >> 6], 1ULL << (s & 63));
  if (e < w.nb)
    atomicOr((unsigned long long*)&docmask[e >> 6], 1ULL << (e & 63));
  atomicOr((unsigned long long*)&w.lits[s >> 6], 1ULL << (s & 63));
  for (int64_t q = s + 1; q < e;) {  // litb: bits s+1 .. e-1, word by word
    const int64_t wd = q >> 6, hi = (wd + 1) * 64 < e ? (wd + 1) * 64 : e;
    const int lo_b = (int)(q & 63), n = (int)(hi - q);
    const uint64_t m = n >= 64 ? ~0ULL : (((1ULL << n) - 1) << lo_b);
    atomicOr((unsigned long long*)&w.litb[wd], m);
    q = hi;
  }
  w.tok[s] = a.id[lit];
  for (int64_t q = s + 1; q < e; ++q) w.tok[q] = INVALID_ID;
  atomicAdd(w.nlit, 1u);
}

// One thread per mask word. Each certain candidate in the word is chosen,
// and its thread walks on through the candidates after it, each within
// lmax - 1 bytes of the one before, up to the next certain one: a candidate
// there is chosen when it starts at or after the end of the last choice (a
// literal chosen before the certain candidate cannot reach past it, or the
// candidate would not be certain). Every walk is finite: candidates only
// grow along it.
__global__ __launch_bounds__(256) void k_added_select(DevAdded a, DevWork w,
                                                      uint64_t* docmask,
                                                      int64_t nwords) {
  const int64_t wd = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (wd >= nwords) return;
  uint64_t m = w.cand[wd];
  const int64_t L = a.lmax;
  while (m) {
    const int64_t p = wd * 64 + __builtin_ctzll(m);
    m &= m - 1;
    if (!certain(a, w, p)) continue;
    choose(a, w, docmask, p);
    int64_t cover = p + a.len[w.litm[p]], prev = p;
    for (;;) {
      // a candidate lmax or more bytes after the last one is certain
      const int64_t q = next_cand(w.cand, prev, prev + L, nwords);
      if (q < 0 || certain(a, w, q)) break;
      if (q >= cover) {
        choose(a, w, docmask, q);
        cover = q + a.len[w.litm[q]];
      }
      prev = q;
    }
  }
}

}  // namespace

hipError_t launch_added(const DevAdded& a, const DevWork& w, bool clear_docmask,
                        hipStream_t s, hipEvent_t start) {
  const int64_t nwords = (w.nb + 63) / 64 + 2;  // the words k_pretok reads
  uint64_t* dm = const_cast<uint64_t*>(w.docmask);
  const uint32_t gf = (uint32_t)((nwords * 64 + ADDED_BLOCK_BYTES - 1) / ADDED_BLOCK_BYTES);
  if (start)
    hipExtLaunchKernelGGL(k_added_find, dim3(gf), dim3(256), 0, s, start,
                          nullptr, 0, a, w, dm, clear_docmask ? 1 : 0, nwords);
  else
    hipLaunchKernelGGL(k_added_find, dim3(gf), dim3(256), 0, s, a, w, dm,
                       clear_docmask ? 1 : 0, nwords);
  const uint32_t gs = (uint32_t)((nwords + 255) / 256);
  hipLaunchKernelGGL(k_added_select, dim3(gs), dim3(256), 0, s, a, w, dm, nwords);
  return hipGetLastError();
}

}  // namespace tk
