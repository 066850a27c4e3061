// tk_device.hip -- gfx950 kernels of the fresh-encode path.
//
// Stages (one stream; the long-piece stages on a second one, beside stage 2):
//   1. k_pretok       per byte: UTF-8 validation, class lookup, NFC quick
//                     check, and the family split rules as a per-character
//                     piece-start predicate -> one start bit per byte.
//      (k_pretok also sizes the pieces that start in its tile: pieces of
//                     1-2 bytes are finished there, longer than 64 queued
//                     for stage 3, the rest listed by length class.)
//   2. k_bpe_pack     merges the listed pieces of 2..64 bytes (lowest rank
//                     pair, leftmost first), one wave per work unit of one
//                     length class: a piece per lane, per four lanes, or
//                     (lane = byte) per slot of lanes; and, first, the long
//                     pieces of up to 128 bytes, one wave each, state in
//                     registers (wave_bpe_rows).
//   3. longer pieces  (side streams): up to 256 bytes merged whole, one
//                     wave each, state in registers (k_bpe_rows), up to 512
//                     in LDS (k_bpe_wide); longer ones are cut into short
//                     segments at likely token boundaries (k_long_windows),
//                     merged segment by segment with boundary-token
//                     histories (k_long_segments), and every cut is
//                     certified (k_certify); failed cuts are removed and the
//                     affected segments redone until every cut holds.
//   4. k_compact      device-wide compaction of the per-byte token slots
//                     into the contiguous id buffer, one pass (look-back).
// Token j of a piece is stored at the byte where that token starts, so the
// id order is the byte order and stage 4 needs no per-piece counts.
//
// Split semantics follow the family regexes alternative by alternative
// (Qwen2 / Llama-3: crates/toktier-gigatoken-core/src/pretokenize/
// options.rs:125,:131; GPT-2: options.rs:118), restated per character in
// the way src/toktier/kernels/pretok_kernel.cu:8-27 describes for the
// cl100k rules; the r50k and deepseek predicates are this project's own
// derivations (deepseek: the three Split stages of
// pretok_classes_deepseek.v1.meta.json "patterns" as one per-character rule
// with the stage-1 / stage-2 pieces as regions, checked against the
// sequential restatement by brute force over short strings).
// BPE semantics: HF tokenizers 0.22.2 (lowest rank first, leftmost on
// ties; pretok_kernel.cu:872-881); table formats: bpe_tables.py:99-132.
#include "tk_device.h"

#include <hip/hip_ext.h>

#include <mutex>
#include <type_traits>

namespace tk {

constexpr uint8_t CP_ = 0, CL_ = 1, CN_ = 2, CS_ = 3;
// DeepSeek's seven classes (pretok_classes_deepseek.v1.meta.json "enum")
constexpr uint8_t DS_O = 0, DS_L = 1, DS_M = 2, DS_N = 3, DS_PS = 4,
                  DS_WS = 5, DS_CR = 6;
constexpr int RS_DEEPSEEK = 3;

// ------------------------------------------------------------ helpers

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ULL;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
  return x ^ (x >> 31);
}

// rank<<32 | merged id, or ~0 when the pair has no merge rule: the
// compact two-choice table when the engine built one (tk_device.h), else
// the interleaved boundary table.
__device__ __forceinline__ uint64_t pair_lookup(const DevTables& t,
                                                uint32_t l, uint32_t r) {
  if (t.ctab) {
    if ((l | r) >= (1u << 18)) return ~0ULL;  // every rule's ids fit 18 bits
    const uint64_t x = pair_perm(l, r);
    const uint32_t b1 = (uint32_t)(x & t.cmask);
    const uint32_t tag = (uint32_t)(x >> t.cbits);
    const uint32_t b2 = pair_alt(b1, tag, t.cbits);
    const ulonglong2* tab = reinterpret_cast<const ulonglong2*>(t.ctab);
    const ulonglong2 u = tab[b1], v = tab[b2];  // independent loads
    const uint64_t w0 = (uint64_t)tag << 1, w1 = w0 | 1;
    const uint64_t s = (u.x >> 37) == w0 ? u.x : (u.y >> 37) == w0 ? u.y
                     : (v.x >> 37) == w1 ? v.x : (v.y >> 37) == w1 ? v.y
                     : ~0ULL;
    if (s == ~0ULL) return ~0ULL;
    return (((s >> 18) & 0x7FFFF) << 32) | (s & 0x3FFFF);
  }
  const uint64_t key = ((uint64_t)l << 32) | r;
  uint64_t i = splitmix64(key) & t.pair_mask;
  for (;;) {
    const ulonglong2 s = t.pairs[i];
    if (s.x == key) return s.y;
    if (s.x == ~0ULL) return ~0ULL;
    i = (i + 1) & t.pair_mask;
  }
}

// The compact table's lookup in 32-bit arithmetic (the same key bijection,
// buckets and slot layout as pair_lookup): true, with the merge's rank and
// id, when the pair has a rule. Both candidate buckets are loaded before
// either is inspected (one memory round trip). l, r < 2^18: the engine
// builds the table only when every byte id and every rule id is below 2^18.
__device__ __forceinline__ bool ctab_find(const DevTables& t, uint32_t l,
                                          uint32_t r, uint32_t* rank,
                                          uint32_t* id) {
  const uint32_t a = l;
  const uint32_t b = (r ^ pair_round(l, 0x9E3779u)) & 0x3FFFFu;
  // the 36-bit key a << 18 | b as hi:lo
  const uint32_t lo = (a << 18) | b, hi = a >> 14;
  const uint32_t b1 = lo & (uint32_t)t.cmask;
  const uint32_t tag = __builtin_amdgcn_alignbit(hi, lo, t.cbits);
  const uint32_t b2 = pair_alt(b1, tag, t.cbits);
  const uint4* tab = reinterpret_cast<const uint4*>(t.ctab);
  uint4 u = tab[b1], v = tab[b2];
  // Every word of both buckets is taken here: left to itself the compiler
  // loads the high words first and the low ones only once a tag matched,
  // two dependent memory round trips instead of one.
  asm volatile("" : "+v"(u.x), "+v"(u.y), "+v"(u.z), "+v"(u.w), "+v"(v.x),
               "+v"(v.y), "+v"(v.z), "+v"(v.w));
  // a slot's high word >> 5 is tag << 1 | (second bucket)
  const uint32_t w0 = tag << 1, w1 = w0 | 1u;
  // (masks rather than selects: the slot words are picked with no branch,
  // so the compiler keeps the two 16-byte loads whole)
  const uint32_t k0 = (u.y >> 5) == w0 ? ~0u : 0u, k1 = (u.w >> 5) == w0 ? ~0u : 0u;
  const uint32_t k2 = (v.y >> 5) == w1 ? ~0u : 0u, k3 = (v.w >> 5) == w1 ? ~0u : 0u;
  const uint32_t slo = (u.x & k0) | (u.z & k1) | (v.x & k2) | (v.z & k3);
  const uint32_t shi = (u.y & k0) | (u.w & k1) | (v.y & k2) | (v.w & k3);
  *rank = __builtin_amdgcn_alignbit(shi, slo, 18) & 0x7FFFFu;
  *id = slo & 0x3FFFFu;
  return (k0 | k1 | k2 | k3) != 0u;
}

// The hot-pair table's probe (ctab_find's, over HOT_BITS buckets in LDS):
// true, with the rule, when the pair has a rule of rank < hot_k; false
// says nothing about rules of higher rank (the caller asks the compact
// table then).
__device__ __forceinline__ bool hot_find(const uint4* hot, uint32_t hot_k,
                                         uint32_t l, uint32_t r,
                                         uint32_t* rank, uint32_t* id) {
  const uint32_t b = (r ^ pair_round(l, 0x9E3779u)) & 0x3FFFFu;
  const uint32_t lo = (l << 18) | b, hi = l >> 14;
  const uint32_t b1 = lo & ((1u << HOT_BITS) - 1);
  const uint32_t tag = __builtin_amdgcn_alignbit(hi, lo, HOT_BITS);
  const uint32_t b2 = pair_alt(b1, tag, HOT_BITS);
  const uint4 u = hot[b1], v = hot[b2];
  const uint32_t w0 = tag << 1, w1 = w0 | 1u;
  const uint32_t k0 = (u.y >> 5) == w0 ? ~0u : 0u, k1 = (u.w >> 5) == w0 ? ~0u : 0u;
  const uint32_t k2 = (v.y >> 5) == w1 ? ~0u : 0u, k3 = (v.w >> 5) == w1 ? ~0u : 0u;
  const uint32_t slo = (u.x & k0) | (u.z & k1) | (v.x & k2) | (v.z & k3);
  const uint32_t shi = (u.y & k0) | (u.w & k1) | (v.y & k2) | (v.w & k3);
  *rank = __builtin_amdgcn_alignbit(shi, slo, 18) & 0x7FFFFu;
  *id = slo & 0x3FFFFu;
  return (k0 | k1 | k2 | k3) != 0u && *rank < hot_k;
}

// The block's LDS copy of the hot-pair table (HOT_BYTES at `dst`), filled
// by all threads; the caller synchronizes before the first probe.
__device__ __forceinline__ void hot_stage(const DevTables& t, uint4* dst) {
  const uint4* src = reinterpret_cast<const uint4*>(t.hot);
  for (uint32_t j = threadIdx.x; j < HOT_BYTES / 16; j += blockDim.x) dst[j] = src[j];
}

// whole-piece vocabulary id (ignore_merges) or -1; a piece longer than the
// longest vocabulary entry is none (no hash over it)
__device__ int32_t vocab_lookup(const DevTables& t, const uint8_t* s,
                                int64_t m) {
  if (m > (int64_t)t.vocab_max_len) return -1;
  uint64_t h = 0xCBF29CE484222325ULL;
  for (int64_t j = 0; j < m; ++j) h = (h ^ s[j]) * 0x100000001B3ULL;
  uint64_t i = splitmix64(h) & t.vocab_mask;
  for (;;) {
    const ulonglong2 e = t.vocab[i];
    if (e.x == ~0ULL) return -1;
    if (e.x == h) {
      const int64_t len = (int64_t)((e.y >> 20) & 0x3FF);
      const uint64_t off = e.y >> 30;
      if (len == m) {
        bool eq = true;
        for (int64_t j = 0; j < m && eq; ++j) eq = t.blob[off + j] == s[j];
        if (eq) return (int32_t)(e.y & 0xFFFFF);
      }
    }
    i = (i + 1) & t.vocab_mask;
  }
}

// A device-side repair pass runs only when the pass before it failed cuts.
__device__ __forceinline__ bool pass_live(const DevWork& w) {
  return !w.nfail_prev ||
         __hip_atomic_load(w.nfail_prev, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// the wave's index in its block, as a wave-uniform (scalar) value
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

__device__ __forceinline__ uint64_t mask_le(int lane) {
  return lane == 63 ? ~0ULL : ((2ULL << lane) - 1);
}

__device__ __forceinline__ uint64_t lanes_in(int lo, int hi) {  // [lo, hi)
  const uint64_t up = hi >= 64 ? ~0ULL : ((1ULL << hi) - 1);
  return up & ~((1ULL << lo) - 1);
}

__device__ __forceinline__ void push_pair(uint32_t* list, uint32_t* count,
                                          uint32_t cap, uint32_t* status,
                                          int64_t a, int64_t b) {
  const uint32_t k = atomicAdd(count, 1u);
  if (k < cap) {
    list[2 * k] = (uint32_t)a;
    list[2 * k + 1] = (uint32_t)b;
  } else {
    atomicOr(status, ST_LONGOVF);
  }
}

// ---- piece classes (stage 2)
// A piece is finished without BPE when it is one byte, or two bytes and no
// whole-piece vocabulary rule applies; pieces of 2..64 bytes are merged in
// packed waves by length class; longer ones take the long-piece stages.
constexpr int PIECE_NONE = -1, PIECE_ONE = -2, PIECE_TWO = -3, PIECE_LONG = -4;

__constant__ uint32_t PACK_LOCAL_OFF[PACK_CLASSES] = {
    pack_local_off(0), pack_local_off(1), pack_local_off(2),
    pack_local_off(3), pack_local_off(4), pack_local_off(5),
    pack_local_off(6), pack_local_off(7), pack_local_off(8),
    pack_local_off(9), pack_local_off(10), pack_local_off(11),
    pack_local_off(12)};
static_assert(PACK_CLASSES == 13, "PACK_LOCAL_OFF lists every class");

__device__ __forceinline__ int pack_class(int L) {  // 2 <= L <= 64
  return (L > 2) + (L > 3) + (L > 4) + (L > 5) + (L > 6) + (L > 7) + (L > 8) +
         (L > 10) + (L > 12) + (L > 16) + (L > 21) + (L > 32);
}

// Kind of the piece that starts at bit `lane` of a start word (given the
// word after it): PIECE_NONE if no piece starts there.
__device__ __forceinline__ int piece_kind(uint64_t word, uint64_t next,
                                          int lane, bool two_direct) {
  if (!((word >> lane) & 1)) return PIECE_NONE;
  const uint64_t gt = word & ~mask_le(lane);
  const int L = gt ? __builtin_ctzll(gt) - lane
              : next ? 64 - lane + __builtin_ctzll(next) : 65;
  if (L == 1) return PIECE_ONE;
  if (L == 2 && two_direct) return PIECE_TWO;
  if (L <= 64) return pack_class(L);
  return PIECE_LONG;
}

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = __shfl_up(v, d);
    if (lane >= d) v += o;
  }
  return v;
}

__device__ __forceinline__ bool is_cont(uint8_t b) { return (b & 0xC0) == 0x80; }
__device__ __forceinline__ bool crlf(int32_t c) { return c == 10 || c == 13; }
__device__ __forceinline__ int fold(int32_t c) {
  if (c >= 'A' && c <= 'Z') return c + 32;
  if (c == 0x17F) return 's';
  return c;
}

// Decode the character whose first bytes are b0..b3, `avail` of them inside
// the text. *ok is false for any invalid form; the value is then U+FFFD.
__device__ __forceinline__ int32_t decode4(uint32_t b0, uint32_t b1,
                                           uint32_t b2, uint32_t b3,
                                           int64_t avail, bool* ok) {
  int need;
  uint32_t v;
  if (b0 < 0x80) { *ok = true; return (int32_t)b0; }
  if (b0 < 0xC0) { *ok = false; return 0xFFFD; }
  if (b0 < 0xE0) { need = 1; v = b0 & 0x1F; }
  else if (b0 < 0xF0) { need = 2; v = b0 & 0x0F; }
  else if (b0 < 0xF8) { need = 3; v = b0 & 0x07; }
  else { *ok = false; return 0xFFFD; }
  for (int k = 1; k <= need; ++k) {
    const uint32_t x = k == 1 ? b1 : k == 2 ? b2 : b3;
    if (k >= avail || (x & 0xC0) != 0x80) { *ok = false; return 0xFFFD; }
    v = (v << 6) | (x & 0x3F);
  }
  if ((need == 1 && v < 0x80) || (need == 2 && v < 0x800) ||
      (need == 3 && v < 0x10000) || v > 0x10FFFF ||
      (v >= 0xD800 && v <= 0xDFFF)) {
    *ok = false;
    return 0xFFFD;
  }
  *ok = true;
  return (int32_t)v;
}

struct Ch {
  int64_t pos;
  int32_t cp;
  uint8_t cl;
};

// Positions are byte offsets into the request; a character is named by the
// byte where it starts. A context answers four questions for the split
// predicates: does a document start at i, where does the previous / next
// character start, which character (code point, class) is at p.
// GCtx reads the request in HBM.
struct GCtx {
  const uint8_t* t;
  int64_t nb;
  const uint64_t* dm;  // document-start bits or nullptr
  const uint8_t* cls;

  __device__ __forceinline__ bool ds(int64_t i) const {
    if (i == 0) return true;
    // read as a 32-bit half: a load the compiler cannot merge with the
    // 64-bit reads of the staged words (that merge makes a flat load, which
    // waits for every memory operation in flight)
    return dm && ((reinterpret_cast<const uint32_t*>(dm)[i >> 5] >> (i & 31)) & 1);
  }
  __device__ __forceinline__ int32_t cp_at(int64_t i, bool* ok) const {
    const int64_t a = nb - i;
    return decode4(t[i], a > 1 ? t[i + 1] : 0, a > 2 ? t[i + 2] : 0,
                   a > 3 ? t[i + 3] : 0, a, ok);
  }
  __device__ __forceinline__ Ch at(int64_t p) const {
    bool ok;
    const int32_t cp = cp_at(p, &ok);
    return Ch{p, cp, cls[cp]};
  }
  // start of the character before the one at p; -1 if p starts a document
  __device__ __forceinline__ int64_t prev(int64_t p) const {
    if (ds(p)) return -1;
    int64_t q = p - 1;
    int k = 0;
    while (q > 0 && k < 3 && is_cont(t[q])) { --q; ++k; }
    return q;
  }
  // start of the character after the one at p; -1 at text / document end
  __device__ __forceinline__ int64_t next(int64_t p) const {
    int64_t q = p + 1;
    int k = 0;
    while (q < nb && k < 3 && is_cont(t[q])) { ++q; ++k; }
    if (q >= nb || ds(q)) return -1;
    return q;
  }
};

// Pretokenize tiles: a block stages PT_TILE bytes plus PT_PAD bytes each
// side in LDS and decodes one entry per byte position for the tile plus
// PT_HALO positions each side:
//   bits  0..20 code point (decode at that byte; U+FFFD if invalid there)
//   bits 21..22 class (bits 0..1)
//   bits 23..24 back: prev(p) = p - 1 - back(p - 1)
//   bits 25..26 fwd:  next(p) = p + 1 + fwd(p) (before the end checks)
//   bit  27     the decode at p is valid UTF-8
//   bits 28..29 class bits 2..3 (the seven DeepSeek / o200k classes, the
//               ten kimi classes)
//   bits 30..31 back(p - 1), so that prev(p) = p - 1 - (entry(p) >> 30)
//               reads the entry at p only (set at every span position)
// packed LDS table entry of k_pretok: byte id (LTAB_NOID: none), class of
// the code point, its NFC quick-check value
constexpr uint32_t LTAB_NOID = 0xFFFFFu;
constexpr int LTAB_CLS = 20, LTAB_NFC = 24;
// a tile's digit-run word (nrun): call tag << 32 | NRUN_FULL (the run
// spans the whole tile) | N characters of the run at the tile's end
constexpr uint64_t NRUN_FULL = 1ull << 31;
// A wait on another workgroup's published word ends at a deadline on the
// device's constant-rate real-time counter, DevWork::wait_ticks after the
// waiting workgroup's first poll: far above any launch's duration, so only
// a broken protocol reaches it, and the call then fails with the stage
// named (ST_STALL_PRETOK, ST_STALL) instead of hanging.
struct WaitBound {
  uint64_t end = 0;  // 0: not started
  __device__ __forceinline__ bool expired(uint64_t ticks) {
    const uint64_t now = (uint64_t)wall_clock64();
    if (end == 0) {
      end = now + ticks;
      return false;
    }
    return now > end;
  }
};
__device__ __forceinline__ void nrun_store(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t nrun_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
constexpr int PT_HALO = 64;
constexpr int PT_SPAN = PT_TILE + 2 * PT_HALO;
constexpr int PT_PAD = 80;  // >= PT_HALO + 4, a multiple of 16
constexpr int PT_BYTES = PT_TILE + 2 * PT_PAD;
constexpr int PT_DMW = PT_TILE / 64 + 6;  // doc-mask words from tile word - 3

// LCtx answers from a block's LDS tile and falls back to GCtx for
// positions outside it (long digit / whitespace runs, rare).
struct LCtx {
  GCtx g;
  const uint32_t* se;  // entries of positions [lo, lo + PT_SPAN)
  int64_t lo;
  const uint64_t* sdm;  // doc-mask words [wlo, wlo + PT_DMW)
  int64_t wlo;

  __device__ __forceinline__ bool in(int64_t p) const {
    return (uint64_t)(p - lo) < (uint64_t)PT_SPAN;
  }
  __device__ __forceinline__ bool ds(int64_t i) const {
    if (i == 0) return true;
    if (!g.dm) return false;
    const int64_t k = (i >> 6) - wlo;
    if ((uint64_t)k < (uint64_t)PT_DMW) return (sdm[k] >> (i & 63)) & 1;
    return g.ds(i);
  }
  __device__ __forceinline__ Ch at(int64_t p) const {
    if (!in(p)) return g.at(p);
    const uint32_t e = se[p - lo];
    return Ch{p, (int32_t)(e & 0x1FFFFF), (uint8_t)(((e >> 21) & 3) | ((e >> 26) & 0xC))};
  }
  __device__ __forceinline__ int64_t prev(int64_t p) const {
    if (ds(p)) return -1;
    const int64_t q = p - 1;
    if (!in(q)) return g.prev(p);
    return q - ((se[q - lo] >> 23) & 3);
  }
  __device__ __forceinline__ int64_t next(int64_t p) const {
    if (!in(p)) return g.next(p);
    const int64_t q = p + 1 + ((se[p - lo] >> 25) & 3);
    if (q >= g.nb || ds(q)) return -1;
    return q;
  }
};

// Is the apostrophe (or other P char) at q the start of a regex match?
// It is unless it continues a P run or follows a U+0020 that the
// " ?[^\s\p{L}\p{N}]+" alternative takes with it.
template <class C>
__device__ __forceinline__ bool p_arrives(const C& c, int64_t q) {
  const int64_t r = c.prev(q);
  if (r < 0) return true;
  const Ch x = c.at(r);
  return x.cl != CP_ && x.cp != ' ';
}

// ---- cl100k (Qwen2 / Llama-3) piece-start predicate for a character
// that does not start a document.
template <class C>
__device__ bool start_cl100k(const C& c, const Ch& ci, int dmax) {
  const Ch p1 = c.at(c.prev(ci.pos));
  if (ci.cl == CN_) {
    // \p{N}{1,K}: digit runs split into groups of K from the run start
    if (dmax <= 1) return true;
    int64_t n = 0;
    for (int64_t q = ci.pos;;) {
      const int64_t r = c.prev(q);
      if (r < 0 || c.at(r).cl != CN_) break;
      ++n;
      q = r;
    }
    return n % dmax == 0;
  }
  if (ci.cl == CL_) {
    if (p1.cl != CL_) {
      // run head: taken by the preceding char as the optional prefix of
      // [^\r\n\p{L}\p{N}]?\p{L}+ (non-CR/LF whitespace, or a single P
      // char that starts its own match -- the contraction alternative
      // consumes the letter just as well)
      if (p1.cl == CS_) return crlf(p1.cp);
      if (p1.cl == CP_) return !p_arrives(c, p1.pos);
      return true;
    }
    // inside a letter run: only a contraction match can end here
    const int64_t q2 = c.prev(p1.pos);
    if (q2 < 0) return false;
    const Ch p2 = c.at(q2);
    if (p2.cp == '\'') {
      const int f1 = fold(p1.cp);
      return (f1 == 's' || f1 == 't' || f1 == 'm' || f1 == 'd') &&
             p_arrives(c, q2);
    }
    if (p2.cl != CL_) return false;
    const int64_t q3 = c.prev(q2);
    if (q3 < 0) return false;
    if (c.at(q3).cp != '\'') return false;
    const int f1 = fold(p2.cp), f2 = fold(p1.cp);
    return ((f1 == 'r' && f2 == 'e') || (f1 == 'v' && f2 == 'e') ||
            (f1 == 'l' && f2 == 'l')) &&
           p_arrives(c, q3);
  }
  if (ci.cl == CP_) return p1.cl != CP_ && p1.cp != ' ';
  // whitespace
  const bool cr_i = crlf(ci.cp);
  if (p1.cl != CS_) return !(p1.cl == CP_ && cr_i);  // [\r\n]* absorption
  const bool cr_1 = crlf(p1.cp);
  if (cr_1 && !cr_i) {
    // right after the last CR/LF of the run (end of \s*[\r\n]+) ...
    bool more = false;
    for (int64_t q = c.next(ci.pos); q >= 0; q = c.next(q)) {
      const Ch x = c.at(q);
      if (x.cl != CS_) break;
      if (crlf(x.cp)) { more = true; break; }
    }
    if (!more) return true;
    // ... or the first char the P match's [\r\n]* left over
    for (int64_t q = p1.pos;;) {
      const int64_t r = c.prev(q);
      if (r < 0) return false;
      const Ch x = c.at(r);
      if (x.cl != CS_) return x.cl == CP_;
      if (!crlf(x.cp)) return false;
      q = r;
    }
  }
  if (!cr_1 && !cr_i) {
    // \s+(?!\S) backs off one char before a non-space (not at text end)
    const int64_t q = c.next(ci.pos);
    return q >= 0 && c.at(q).cl != CS_;
  }
  return false;
}

// ---- r50k (GPT-2) piece-start predicate.
template <class C>
__device__ bool start_r50k(const C& c, const Ch& ci) {
  const Ch p1 = c.at(c.prev(ci.pos));
  if (ci.cl == CS_) {
    if (p1.cl != CS_) return true;
    const int64_t q = c.next(ci.pos);
    return q >= 0 && c.at(q).cl != CS_;
  }
  if (ci.cl == CN_ || ci.cl == CP_) {
    if (p1.cl == ci.cl) return false;
    return p1.cp != ' ';
  }
  if (p1.cl != CL_) {
    if (p1.cp == ' ') return false;
    if (p1.cp == '\'' && p_arrives(c, p1.pos)) {
      const int a = ci.cp;
      if (a == 's' || a == 't' || a == 'm' || a == 'd') return false;
      const int64_t qn = c.next(ci.pos);
      if (qn >= 0) {
        const int b = c.at(qn).cp;
        if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') ||
            (a == 'l' && b == 'l'))
          return false;
      }
    }
    return true;
  }
  const int64_t q2 = c.prev(p1.pos);
  if (q2 < 0) return false;
  const Ch p2 = c.at(q2);
  if (p2.cp == '\'') {
    const int a = p1.cp;
    return (a == 's' || a == 't' || a == 'm' || a == 'd') && p_arrives(c, q2);
  }
  if (p2.cl != CL_) return false;
  const int64_t q3 = c.prev(q2);
  if (q3 < 0 || c.at(q3).cp != '\'') return false;
  const int a = p2.cp, b = p1.cp;
  return ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') ||
          (a == 'l' && b == 'l')) &&
         p_arrives(c, q3);
}

// ---- the same predicates from a fixed context, without branches on
// loads: the character (c0), the four before it (c1..c4, nearest first;
// hN false where the text or document ends) and the one after it (cn, hn).
// Returns 1 (starts a piece), 0, or, when the answer needs more of the
// run around the character: FAST_DIGITS (the digits before it decide,
// group width over 1) or FAST_CRLF (whitespace right after a CR/LF: the
// rest of the whitespace run decides).
constexpr int FAST_DIGITS = -2, FAST_CRLF = -3;
struct Ctx5 {
  uint32_t c0, c1, c2, c3, c4, cn;  // entries (code point | class << 21)
  bool h2, h3, h4, hn;              // c1 always exists
};
__device__ __forceinline__ int ecl(uint32_t e) { return (e >> 21) & 3; }
__device__ __forceinline__ int ecp(uint32_t e) { return (int)(e & 0x1FFFFF); }
// p_arrives of the character whose predecessor is e (present: h)
__device__ __forceinline__ bool arrives_after(uint32_t e, bool h) {
  return !h || (ecl(e) != CP_ && ecp(e) != ' ');
}
__device__ __forceinline__ bool is_stmd(int f) {
  return f == 's' || f == 't' || f == 'm' || f == 'd';
}
__device__ __forceinline__ bool is_re_ve_ll(int a, int b) {
  return (a == 'r' && b == 'e') || (a == 'v' && b == 'e') ||
         (a == 'l' && b == 'l');
}

__device__ __forceinline__ int fast_cl100k(const Ctx5& x, int dmax) {
  const int k0 = ecl(x.c0), k1 = ecl(x.c1);
  const int k2 = x.h2 ? ecl(x.c2) : -1, k3 = x.h3 ? ecl(x.c3) : -1;
  if (k0 == CN_) {
    if (dmax <= 1) return 1;
    // digits before this one: 0, 1 or 2 decide; 3 or more need the run
    if (k1 != CN_) return 1;
    if (k2 != CN_) return 1 % dmax == 0;
    if (k3 != CN_) return 2 % dmax == 0;
    return FAST_DIGITS;
  }
  const int p1 = ecp(x.c1);
  if (k0 == CL_) {
    if (k1 != CL_) {
      if (k1 == CS_) return crlf(p1);
      if (k1 == CP_) return !arrives_after(x.c2, x.h2);
      return 1;
    }
    const int p2 = x.h2 ? ecp(x.c2) : -1;
    if (p2 == '\'') return is_stmd(fold(p1)) && arrives_after(x.c3, x.h3);
    if (k2 != CL_) return 0;
    const int p3 = x.h3 ? ecp(x.c3) : -1;
    return p3 == '\'' && is_re_ve_ll(fold(p2), fold(p1)) &&
           arrives_after(x.c4, x.h4);
  }
  if (k0 == CP_) return k1 != CP_ && p1 != ' ';
  const bool cr_i = crlf(ecp(x.c0));
  if (k1 != CS_) return !(k1 == CP_ && cr_i);
  const bool cr_1 = crlf(p1);
  if (cr_1 && !cr_i) return FAST_CRLF;
  if (!cr_1 && !cr_i) return x.hn && ecl(x.cn) != CS_;
  return 0;
}

__device__ __forceinline__ int fast_r50k(const Ctx5& x) {
  const int k0 = ecl(x.c0), k1 = ecl(x.c1), p0 = ecp(x.c0), p1 = ecp(x.c1);
  if (k0 == CS_) return k1 != CS_ || (x.hn && ecl(x.cn) != CS_);
  if (k0 == CN_ || k0 == CP_) return k1 != k0 && p1 != ' ';
  if (k1 != CL_) {
    if (p1 == ' ') return 0;
    if (p1 == '\'' && arrives_after(x.c2, x.h2)) {
      if (is_stmd(p0)) return 0;
      if (x.hn && is_re_ve_ll(p0, ecp(x.cn))) return 0;
    }
    return 1;
  }
  const int p2 = x.h2 ? ecp(x.c2) : -1;
  if (p2 == '\'') return is_stmd(p1) && arrives_after(x.c3, x.h3);
  if (!x.h2 || ecl(x.c2) != CL_) return 0;
  const int p3 = x.h3 ? ecp(x.c3) : -1;
  return p3 == '\'' && is_re_ve_ll(p2, p1) && arrives_after(x.c4, x.h4);
}

// ---- DeepSeek (DeepSeek V3 / V4) piece-start predicate. Three Split
// stages run in order: \p{N}{1,3}; the CJK-range runs
// [一-龥぀-ゟ゠-ヿ]+; then
// [ascii punct][A-Za-z]+|[^\r\n\p{L}\p{P}\p{S}]?[\p{L}\p{M}]+
// | ?[\p{P}\p{S}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+ inside each piece, the
// spans it does not match kept as pieces. The stage-1 and stage-2 pieces
// are regions: digits (grouped by 3 from the run start), CJK-range runs,
// and the rest. A region change starts a piece, and the stage-3 rule reads
// no character across one (a region end is an end of text to it). Inside a
// region, with p1 the character before c0 in it:
//   c0 letter / mark: after a letter / mark, only where an ASCII-alpha run
//     that [ascii punct][A-Za-z]+ took ends (c0 not ASCII alpha, p1 is, and
//     the run is led by an ASCII punct that starts its own match); after P
//     or S unless c0 is ASCII alpha taken by that alternative; after CR/LF
//   c0 P / S: unless p1 is P / S (the run) or U+0020 (" ?" takes it)
//   c0 CR/LF: after a letter, mark or other (O) character
//   c0 O: unless p1 is O and c0 is no match start (none begins at an O
//     character that is not followed by a letter or mark)
//   c0 other whitespace: after a non-space; after whitespace before a
//     non-space (\s+(?!\S) backs off one); right after a CR/LF unless
//     another CR/LF follows in the run and the CR/LF run before c0 was not
//     the [\r\n]* of a P / S match
__device__ __forceinline__ int dcl(uint32_t e) {
  return (int)(((e >> 21) & 3) | ((e >> 26) & 0xC));
}
__device__ __forceinline__ bool ds_cjk(int c) {
  return (c >= 0x4E00 && c <= 0x9FA5) || (c >= 0x3040 && c <= 0x30FF);
}
__device__ __forceinline__ int ds_region(int k, int cp) {
  return k == DS_N ? 2 : ds_cjk(cp) ? 1 : 0;
}
__device__ __forceinline__ bool ascii_punct(int c) {
  return (c >= 0x21 && c <= 0x2F) || (c >= 0x3A && c <= 0x40) ||
         (c >= 0x5B && c <= 0x60) || (c >= 0x7B && c <= 0x7E);
}
__device__ __forceinline__ bool ascii_alpha(int c) {
  return (uint32_t)((c | 32) - 'a') < 26u;
}
__device__ __forceinline__ bool ds_lm(int k) { return k == DS_L || k == DS_M; }
__device__ __forceinline__ bool ds_space(int k) { return k >= DS_WS; }

template <class C>
__device__ bool ds_run_led(const C& c, int64_t s);
// FAST_FAR: a letter / mark after an ASCII-alpha run that reaches below the
// LDS span; *far is the highest position of the run not yet read, and the
// wave searches from there (ds_stop_hbm)
constexpr int FAST_FAR = -5;
template <class C>
__device__ int start_deepseek(const C& c, const Ch& ci, int dmax, int64_t* far) {
  const int r0 = ds_region(ci.cl, ci.cp);
  // the character before / after p inside c0's region (-1 at its edge)
  auto prev_in = [&](int64_t p) -> int64_t {
    const int64_t q = c.prev(p);
    if (q < 0) return -1;
    const Ch x = c.at(q);
    return ds_region(x.cl, x.cp) == r0 ? q : -1;
  };
  auto next_in = [&](int64_t p) -> int64_t {
    const int64_t q = c.next(p);
    if (q < 0) return -1;
    const Ch x = c.at(q);
    return ds_region(x.cl, x.cp) == r0 ? q : -1;
  };
  // does the P/S character at q start its own match
  auto arrives = [&](int64_t q) {
    const int64_t r = prev_in(q);
    if (r < 0) return true;
    const Ch x = c.at(r);
    return x.cl != DS_PS && x.cp != ' ';
  };
  const int64_t q1 = prev_in(ci.pos);
  if (q1 < 0) return true;
  if (ci.cl == DS_N) {
    if (dmax <= 1) return true;
    int64_t n = 0;
    for (int64_t q = q1; q >= 0; q = prev_in(q)) ++n;
    return n % dmax == 0;
  }
  const Ch p1 = c.at(q1);
  if (ds_lm(ci.cl)) {
    if (ds_lm(p1.cl)) {
      if (ascii_alpha(ci.cp) || !ascii_alpha(p1.cp)) return false;
      // down the run (one byte per letter) while it stays in the span
      for (int64_t q = q1;;) {
        if (c.ds(q)) return false;  // a document starts inside the run
        const int64_t r = q - 1;
        if (!c.in(r)) {
          *far = r;
          return FAST_FAR;
        }
        if (!ascii_alpha(c.at(r).cp)) return ds_run_led(c, r);
        q = r;
      }
    }
    if (p1.cl == DS_PS)
      return !(ascii_alpha(ci.cp) && ascii_punct(p1.cp) && arrives(q1));
    return p1.cl == DS_CR;
  }
  if (ci.cl == DS_PS) return p1.cl != DS_PS && p1.cp != ' ';
  if (ci.cl == DS_CR) return ds_lm(p1.cl) || p1.cl == DS_O;
  if (ci.cl == DS_O) {
    if (p1.cl != DS_O) return true;
    const int64_t q = next_in(ci.pos);
    return q >= 0 && ds_lm(c.at(q).cl);
  }
  // other whitespace
  if (!ds_space(p1.cl)) return true;
  if (p1.cl == DS_WS) {
    const int64_t q = next_in(ci.pos);
    return q >= 0 && !ds_space(c.at(q).cl);
  }
  bool more = false;
  for (int64_t q = next_in(ci.pos); q >= 0; q = next_in(q)) {
    const Ch x = c.at(q);
    if (!ds_space(x.cl)) break;
    if (x.cl == DS_CR) { more = true; break; }
  }
  if (!more) return true;
  for (int64_t q = q1;;) {
    const int64_t r = prev_in(q);
    if (r < 0) return false;
    const Ch x = c.at(r);
    if (!ds_space(x.cl)) return x.cl == DS_PS;
    if (x.cl != DS_CR) return false;
    q = r;
  }
}

// The same from the fixed context; FAST_GENERAL: an ASCII-alpha run longer
// than the context, walked by the general predicate.
constexpr int FAST_GENERAL = -4;
__device__ __forceinline__ int fast_deepseek(const Ctx5& x, int dmax) {
  const int k0 = dcl(x.c0), p0 = ecp(x.c0);
  const int k1 = dcl(x.c1), p1 = ecp(x.c1);
  const int r0 = ds_region(k0, p0);
  if (ds_region(k1, p1) != r0) return 1;
  const int k2 = dcl(x.c2), p2 = ecp(x.c2), k3 = dcl(x.c3), p3 = ecp(x.c3);
  const int k4 = dcl(x.c4), p4 = ecp(x.c4), kn = dcl(x.cn);
  // present inside c0's region
  const bool h2 = x.h2 && ds_region(k2, p2) == r0;
  const bool h3 = h2 && x.h3 && ds_region(k3, p3) == r0;
  const bool h4 = h3 && x.h4 && ds_region(k4, p4) == r0;
  const bool hn = x.hn && ds_region(kn, ecp(x.cn)) == r0;
  if (k0 == DS_N) {
    if (dmax <= 1) return 1;
    if (!h2) return 1 % dmax == 0;
    if (!h3) return 2 % dmax == 0;
    return FAST_DIGITS;
  }
  // does a P/S character whose predecessor (present: h) is k, p start a match
  auto arrives = [](bool h, int k, int p) { return !h || (k != DS_PS && p != ' '); };
  if (ds_lm(k0)) {
    if (ds_lm(k1)) {
      if (ascii_alpha(p0) || !ascii_alpha(p1)) return 0;
      if (!h2) return 0;
      if (!ascii_alpha(p2)) return ascii_punct(p2) && arrives(h3, k3, p3);
      if (!h3) return 0;
      if (!ascii_alpha(p3)) return ascii_punct(p3) && arrives(h4, k4, p4);
      return FAST_GENERAL;
    }
    if (k1 == DS_PS) return !(ascii_alpha(p0) && ascii_punct(p1) && arrives(h2, k2, p2));
    return k1 == DS_CR;
  }
  if (k0 == DS_PS) return k1 != DS_PS && p1 != ' ';
  if (k0 == DS_CR) return ds_lm(k1) || k1 == DS_O;
  if (k0 == DS_O) return k1 != DS_O || (hn && ds_lm(kn));
  if (!ds_space(k1)) return 1;
  if (k1 == DS_WS) return hn && !ds_space(kn);
  // right after a CR/LF: a start unless another CR/LF follows in the run
  // and the CR/LF run before c0 is not a P / S match's [\r\n]*
  if (!hn || !ds_space(kn)) return 1;
  if (kn == DS_WS) return FAST_CRLF;
  if (!h2) return 0;
  if (k2 == DS_PS) return 1;
  if (k2 != DS_CR) return 0;
  if (!h3) return 0;
  if (k3 == DS_PS) return 1;
  if (k3 != DS_CR) return 0;
  return FAST_CRLF;
}

// A letter / mark right after an ASCII-alpha run (FAST_GENERAL) starts a
// piece exactly when [ascii punct][A-Za-z]+ took the run: the run holds no
// document start, and the character before it, whose last byte is s, is
// ASCII punctuation that starts its own match (no P/S and no U+0020
// before it in its region, or a document start at s). So the answer needs
// only s, the highest position below the run that is not an ASCII letter
// or that opens a document, however long the run is.
template <class C>
__device__ bool ds_run_led(const C& c, int64_t s) {
  if (s < 0) return false;
  const Ch x = c.at(s);  // (a non-ASCII byte at s gives a code point >= 0x80)
  if (!ascii_punct(x.cp)) return false;
  const int64_t q = c.prev(s);
  if (q < 0) return true;
  const Ch y = c.at(q);
  return ds_region(y.cl, y.cp) != 0 || (y.cl != DS_PS && y.cp != ' ');
}
// The ASCII letters of four bytes, one bit each (bit 7 of every byte);
// no byte carries into the next (every sum stays below 0x100).
__device__ __forceinline__ uint32_t alpha_bytes(uint32_t v) {
  const uint32_t y = (v | 0x20202020u) & 0x7F7F7F7Fu;  // lower case, 7 bits
  const uint32_t ge = y + 0x1F1F1F1Fu;                 // >= 'a'
  const uint32_t gt = y + 0x05050505u;                 // > 'z'
  const uint32_t a = ge & ~gt & ~v & 0x80808080u;      // and ASCII
  return ((a >> 7) & 1u) | ((a >> 14) & 2u) | ((a >> 21) & 4u) | ((a >> 28) & 8u);
}
// Wave-cooperative: the highest position <= q that is not an ASCII letter
// or that opens a document, read from the text in HBM. Lane l takes the
// 64-byte chunk (q >> 6) - l of each 4 KiB step, so a step is one wave of
// coalesced loads; chunk 0 holds position 0, which opens the text, so the
// search ends there at the latest. q >= 0; every lane calls it with the
// same q (wave-uniform).
__device__ int64_t ds_stop_hbm(const uint8_t* t, const uint64_t* dm, int64_t q) {
  const int lane = (int)(threadIdx.x & 63);
  const bool al = ((uintptr_t)t & 15) == 0;
  for (int64_t cq = q >> 6; cq >= 0; cq -= 64) {
    const int64_t ch = cq - lane;
    uint64_t m = 0;
    if (ch >= 0) {
      const uint8_t* p = t + 64 * ch;  // the whole chunk lies at or below q | 63 < nb
      uint64_t alpha = 0;
      if (al) {
        const uint4* v = reinterpret_cast<const uint4*>(p);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint4 x = v[j];
          alpha |= (uint64_t)(alpha_bytes(x.x) | (alpha_bytes(x.y) << 4) |
                              (alpha_bytes(x.z) << 8) | (alpha_bytes(x.w) << 12))
                   << (16 * j);
        }
      } else {
        for (int j = 0; j < 64; ++j) alpha |= (uint64_t)ascii_alpha(p[j]) << j;
      }
      m = ~alpha;
      if (dm) m |= dm[ch];
      if (ch == 0) m |= 1;
      if (ch == (q >> 6)) m &= mask_le((int)(q & 63));
    }
    const uint64_t any = __ballot(m != 0);
    if (any) {
      const int l = __builtin_ctzll(any);
      const int hb = m ? 63 - __builtin_clzll(m) : 0;
      return 64 * (cq - l) + __builtin_amdgcn_readlane(hb, l);
    }
  }
  return -1;  // (q < 0: nothing to search)
}

// ---- o200k (gpt-oss): o200k_base with contractions,
// [^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}]*[\p{Ll}\p{Lm}\p{Lo}\p{M}]+C?
// |[^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}]+[\p{Ll}\p{Lm}\p{Lo}\p{M}]*C?
// |\p{N}{1,K}| ?[^\s\p{L}\p{N}]+[\r\n/]*|\s*[\r\n]+|\s+(?!\S)|\s+
// with C = (?i:'s|'t|'re|'ve|'m|'ll|'d), over the classes P U L C N S M
// (U = Lu Lt, L = Ll, C = Lm Lo; W = U L C M are the letter classes).
// Whether a character starts a piece depends on context of any length to
// its left (a mark continues a P match or a letter match; a run of C
// characters after a lower-case letter is one letter match, after
// anything else it can end before an upper-case run), so the split is a
// left-to-right automaton: the state after each character, one of eight,
// is what the character after it needs. Each character is a transition
// function of the previous state (a byte per state: the functions compose
// by byte permutes) and a start bit per previous state; the functions
// compose by a wave scan, and a tile's entry state comes from the word
// before it or from the tiles before it.
// States (the previous character is ...):
//   PUN   in a P match's [PM]+ (or the U+0020 that opens one)
//   TAIL  in its [\r\n/]* tail
//   LPRE  the prefix character of a letter match (a letter follows)
//   LU    a U letter of a letter match
//   LBL   a B letter (L C M) whose run of B letters since the last U (or
//         the match's first letter) holds an L
//   LBN   a B letter whose run holds no L
//   CONTR a contraction's apostrophe or first letter, more letters follow
//         (the letter's own predecessor tells whether it is the first of
//         two: 're 've 'll)
//   FRESH the match ends after it (digits, the last contraction letter),
//         or it is in a whitespace match (a whitespace character after
//         another one reads it so: no other state follows a whitespace
//         character that a whitespace character can follow)
// Inside a letter run only U letters start pieces: after LBL always (the
// [A]*[B]+ alternative stopped there), after LBN exactly when every
// character from it to the run's end is U (A* gave the run back to its
// last B letter); the letter match's first letter starts at its own
// class state, and a prefix character or mark that opens one changes
// nothing about where it ends.
constexpr int RS_O200K = 4;
constexpr int RS_KIMI = 5;
constexpr uint8_t OK_P = 0, OK_U = 1, OK_L = 2, OK_C = 3, OK_N = 4,
                  OK_S = 5, OK_M = 6, OK_HL = 7, OK_HN = 8, OK_HP = 9;
enum : uint32_t {
  O2_PUN = 0, O2_TAIL, O2_LPRE, O2_LU, O2_LBL, O2_LBN, O2_CONTR, O2_FRESH,
  // (kimi) in a Han run; one or two digits into a \p{N}{1,3} group
  O2_HAN, O2_D1, O2_D2
};
// states of the o200k / kimi automaton, and the 32-bit words of a
// function (a byte per state; kimi's eleven padded to sixteen)
template <int RS> constexpr int o2_nst() { return RS == RS_KIMI ? 11 : 8; }
template <int RS> constexpr int o2_words() { return RS == RS_KIMI ? 4 : 2; }
template <int W> struct O2Fn { uint32_t d[W]; };
template <int W> __device__ __forceinline__ O2Fn<W> o2_rep(uint32_t v) {
  O2Fn<W> f;
#pragma unroll
  for (int k = 0; k < W; ++k) f.d[k] = v * 0x01010101u;
  return f;
}
template <int W> __device__ __forceinline__ O2Fn<W> o2_ident() {
  O2Fn<W> f;
#pragma unroll
  for (int k = 0; k < W; ++k) f.d[k] = 0x03020100u + (uint32_t)k * 0x04040404u;
  return f;
}
template <int W> __device__ __forceinline__ uint32_t o2_at(const O2Fn<W>& f, uint32_t s) {
  uint32_t d = f.d[0];
#pragma unroll
  for (int k = 1; k < W; ++k) d = (s >> 2) == (uint32_t)k ? f.d[k] : d;
  return (d >> (8 * (s & 3))) & 0xFFu;
}
template <int W> __device__ __forceinline__ void o2_set(O2Fn<W>& f, uint32_t s, uint32_t v) {
  f.d[s >> 2] = (f.d[s >> 2] & ~(0xFFu << (8 * (s & 3)))) | (v << (8 * (s & 3)));
}
// a, then b: byte s of the result is b's byte a[s] (v_perm_b32 picks bytes
// 0..7 of its two sources; kimi's states 8..15 come from the second pair)
template <int W>
__device__ __forceinline__ O2Fn<W> o2_then(const O2Fn<W>& a, const O2Fn<W>& b) {
  O2Fn<W> h;
#pragma unroll
  for (int k = 0; k < W; ++k) {
    const uint32_t x = a.d[k];
    const uint32_t lo = __builtin_amdgcn_perm(b.d[1], b.d[0], x);
    if (W == 2) {
      h.d[k] = lo;
    } else {
      const uint32_t hi = __builtin_amdgcn_perm(b.d[W - 1], b.d[W - 2], x ^ 0x08080808u);
      const uint32_t m = ((x >> 3) & 0x01010101u) * 0xFFu;
      h.d[k] = (hi & m) | (lo & ~m);
    }
  }
  return h;
}
template <int RS>
__device__ __forceinline__ bool o2_const(const O2Fn<o2_words<RS>()>& f) {
  const uint32_t r = (f.d[0] & 0xFFu) * 0x01010101u;
  if constexpr (RS == RS_KIMI)
    return f.d[0] == r && f.d[1] == r && ((f.d[2] ^ r) & 0x00FFFFFFu) == 0;
  return f.d[0] == r && f.d[1] == r;
}
// a function as a nibble per state (the tiles' published form) and back
template <int RS> __device__ __forceinline__ uint64_t o2_pack(const O2Fn<o2_words<RS>()>& f) {
  uint64_t x = 0;
#pragma unroll
  for (int s = 0; s < o2_nst<RS>(); ++s) x |= (uint64_t)(o2_at(f, s) & 15u) << (4 * s);
  return x;
}
template <int RS> __device__ __forceinline__ O2Fn<o2_words<RS>()> o2_unpack(uint64_t x) {
  O2Fn<o2_words<RS>()> f = o2_ident<o2_words<RS>()>();
#pragma unroll
  for (int s = 0; s < o2_nst<RS>(); ++s) o2_set(f, s, (uint32_t)(x >> (4 * s)) & 15u);
  return f;
}
// f moved by a DPP control over the wave; lanes with no source (or outside
// the rows of row_mask) get the identity
template <int ctrl, int row_mask, int W>
__device__ __forceinline__ O2Fn<W> o2_dpp(const O2Fn<W>& f) {
  const O2Fn<W> id = o2_ident<W>();
  O2Fn<W> g;
#pragma unroll
  for (int k = 0; k < W; ++k)
    g.d[k] = (uint32_t)__builtin_amdgcn_update_dpp((int)id.d[k], (int)f.d[k], ctrl,
                                                   row_mask, 0xF, false);
  return g;
}
// inclusive composition over the wave's lanes, lane 0 first: within each
// row of 16 (row_shr 1, 2, 4, 8), then rows 1 and 3 after lane 15 of the
// row before (row_bcast:15), rows 2 and 3 after lane 31 (row_bcast:31)
template <int W>
__device__ __forceinline__ O2Fn<W> o2_scan(O2Fn<W> F) {
  F = o2_then(o2_dpp<0x111, 0xF>(F), F);
  F = o2_then(o2_dpp<0x112, 0xF>(F), F);
  F = o2_then(o2_dpp<0x114, 0xF>(F), F);
  F = o2_then(o2_dpp<0x118, 0xF>(F), F);
  F = o2_then(o2_dpp<0x142, 0xA>(F), F);
  F = o2_then(o2_dpp<0x143, 0xC>(F), F);
  return F;
}
template <int W> __device__ __forceinline__ O2Fn<W> o2_lane63(const O2Fn<W>& f) {
  O2Fn<W> g;
#pragma unroll
  for (int k = 0; k < W; ++k) g.d[k] = (uint32_t)__builtin_amdgcn_readlane((int)f.d[k], 63);
  return g;
}
__device__ __forceinline__ bool ok_w(int k) {
  return k == OK_U || k == OK_L || k == OK_C || k == OK_M;
}

// The transition of the character at i: *fo the next state per previous
// state, *go the start bit per previous state (o200k digits: the caller's
// group rule replaces it). x0 is its entry (code point | class), xp / x1
// the entries of the characters before / after it in its document (hp /
// h1: present; d0: a document starts at i). `need_g` false skips what only
// the start bits read; `contr` false drops the contraction suffix (o200k
// rows without it); ws_hint: for a whitespace character right after a
// CR/LF, whether no CR/LF follows in its run (1 / 0, from the word's byte
// masks), -1 when the masks do not tell. The function is built from the
// three entries with selects; the rare cases that read further (an
// upper-case run after a C or M letter, a whitespace run after a CR/LF that
// the masks do not resolve, the second letter of 're 've 'll) walk
// through the context.
// kimi (RS_KIMI): a Han character (HL HN HP) opens or continues a Han run;
// \p{N}{1,3} counts its digits in the state (a Han number inside a group
// is a digit, at a group's start it opens a Han run); P matches take the
// other Han (HP) and their tail is [\r\n]* (no '/').
template <int RS, class C>
__device__ __forceinline__ void o2k_char(const C& c, int64_t i, uint32_t x0, bool d0,
                                         uint32_t xp, bool hp, uint32_t x1, bool h1,
                                         bool need_g, bool contr, int ws_hint,
                                         O2Fn<o2_words<RS>()>* fo, uint32_t* go) {
  constexpr bool KIMI = RS == RS_KIMI;
  constexpr int W = o2_words<RS>();
  constexpr uint32_t ALL = (1u << o2_nst<RS>()) - 1;
  const int32_t cp = ecp(x0), cp1 = ecp(x1), cpp = ecp(xp);
  const int k = dcl(x0);
  const int k1 = h1 ? dcl(x1) : -1, kp = hp ? dcl(xp) : -1;
  const bool cr = crlf(cp);
  const bool han = KIMI && k >= OK_HL;
  const bool w0 = ok_w(k), w1 = ok_w(k1);
  // [^\s\p{L}\p{N}]: the characters a P match's [PM]+ takes
  const bool pm = k == OK_P || k == OK_M || (KIMI && k == OK_HP);
  // the state of a match that starts here
  const bool q0 = k == OK_P || (k == OK_S && !cr);
  const uint32_t ns =
      han ? O2_HAN
      : k == OK_N ? (KIMI ? O2_D1 : O2_FRESH)
      : k == OK_U ? O2_LU
      : k == OK_L ? O2_LBL
      : (k == OK_C || k == OK_M) ? O2_LBN
      : (q0 && w1) ? O2_LPRE
      : (k == OK_P || (cp == ' ' && (k1 == OK_P || (KIMI && k1 == OK_HP)))) ? O2_PUN
      : O2_FRESH;
  O2Fn<W> f = o2_rep<W>(ns);
  uint32_t g = ALL;
  if (d0) {
    *fo = f;
    *go = g;
    return;
  }
  // a P match: [PM]+ goes on, a CR/LF opens the tail
  if (pm || cr) {
    o2_set(f, O2_PUN, pm ? O2_PUN : O2_TAIL);
    g &= ~(1u << O2_PUN);
  }
  if (cr || (!KIMI && cp == '/')) {
    o2_set(f, O2_TAIL, O2_TAIL);
    g &= ~(1u << O2_TAIL);
  }
  if (KIMI) {
    // a Han run goes on; a \p{N} character continues a digit group
    if (han) {
      o2_set(f, O2_HAN, O2_HAN);
      g &= ~(1u << O2_HAN);
    }
    if (k == OK_N || k == OK_HN) {
      o2_set(f, O2_D1, O2_D2);
      o2_set(f, O2_D2, O2_FRESH);
      g &= ~((1u << O2_D1) | (1u << O2_D2));
    }
  }
  if (w0) {
    // a letter after a prefix or inside a letter run (the class state is
    // ns already, except that a C or M letter keeps LBL)
    g &= ~((1u << O2_LPRE) | (1u << O2_LU) | (1u << O2_LBN));
    if (k != OK_U) g &= ~(1u << O2_LBL);
    if (k == OK_C || k == OK_M) o2_set(f, O2_LBL, O2_LBL);
    // a contraction's letters ('s 't 'm 'd: one; 're 've 'll: two): the
    // first of two follows the apostrophe itself
    const int a = fold(cp);
    if (contr && (a == 's' || a == 't' || a == 'm' || a == 'd' || a == 'r' ||
                  a == 'e' || a == 'v' || a == 'l')) {
      const bool two = (a == 'r' || a == 'v' || a == 'l') && hp && cpp == '\'';
      o2_set(f, O2_CONTR, two ? O2_CONTR : O2_FRESH);
      g &= ~(1u << O2_CONTR);
    }
    // after a C or M letter an upper-case letter starts a piece when the
    // U run reaches the letter run's end (LBN is reached only over C or M
    // letters)
    if (need_g && k == OK_U && (kp == OK_C || kp == OK_M)) {
      bool end = !w1;
      if (k1 == OK_U) {
        int64_t q = c.next(c.next(i));
        int kq = q >= 0 ? c.at(q).cl : -1;
        while (q >= 0 && kq == OK_U) {
          q = c.next(q);
          kq = q >= 0 ? c.at(q).cl : -1;
        }
        end = !ok_w(kq);
      }
      if (end) g |= 1u << O2_LBN;
    }
  } else if (contr && cp == '\'' && h1) {
    // a contraction after a letter match
    const int a = fold(cp1);
    bool ap = a == 's' || a == 't' || a == 'm' || a == 'd';
    if (a == 'r' || a == 'v' || a == 'l') {
      const int64_t n2 = c.next(c.next(i));
      if (n2 >= 0) {
        const int b = fold(c.at(n2).cp);
        ap = (a == 'r' && b == 'e') || (a == 'v' && b == 'e') || (a == 'l' && b == 'l');
      }
    }
    if (ap) {
      o2_set(f, O2_LU, O2_CONTR);
      o2_set(f, O2_LBL, O2_CONTR);
      o2_set(f, O2_LBN, O2_CONTR);
      g &= ~((1u << O2_LU) | (1u << O2_LBL) | (1u << O2_LBN));
    }
  }
  if (k == OK_S && kp == OK_S) {
    // after another whitespace character FRESH is the whitespace match:
    // \s*[\r\n]+ ends after the run's last CR/LF; after that (or with
    // none) \s+(?!\S) leaves the run's last character
    bool s = !cr && h1 && k1 != OK_S;
    if (!cr && need_g && crlf(cpp)) {
      // right after a CR/LF: a start unless another CR/LF follows in the
      // run (only the start bit reads this: a start inside the run before
      // its last character leaves FRESH either way)
      s = true;
      if (k1 == OK_S && ws_hint >= 0) {
        s = ws_hint != 0;
      } else if (k1 == OK_S) {
        for (int64_t q = c.next(i); q >= 0;) {
          const Ch x = c.at(q);
          if (x.cl != OK_S) break;
          if (crlf(x.cp)) { s = false; break; }
          q = c.next(q);
        }
      }
    }
    if (!s) {
      o2_set(f, O2_FRESH, O2_FRESH);
      g &= ~(1u << O2_FRESH);
    }
  }
  *fo = f;
  *go = g;
}

// a tile's automaton word pair (ostate[2t], ostate[2t + 1]): call tag << 32
// | the low 32 bits of the tile's function, and call tag << 32 | kind << 30
// | state << 26 | the function's high 20 bits, kind O2_AGG (the function)
// or O2_INCL (the state after the tile)
constexpr uint32_t O2_AGG = 1, O2_INCL = 2;
__device__ __forceinline__ void o2_publish(uint64_t* p, uint32_t seq, uint32_t kind,
                                           uint64_t f, uint32_t s) {
  if (kind == O2_AGG)
    __hip_atomic_store(p, ((uint64_t)seq << 32) | (uint32_t)f, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(p + 1, ((uint64_t)seq << 32) | (kind << 30) | (s << 26) |
                                (uint32_t)((f >> 32) & 0xFFFFF),
                     __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

// exclusive scan of one value per thread over a 256-thread block
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* total) {
  __shared__ uint32_t wsum[4];
  const int lane = threadIdx.x & 63, wv = wave_id();
  const uint32_t inc = wave_incl_scan(v, lane);
  if (lane == 63) wsum[wv] = inc;
  __syncthreads();
  uint32_t off = 0, tot = 0;
  for (int k = 0; k < 4; ++k) {
    if (k < wv) off += wsum[k];
    tot += wsum[k];
  }
  __syncthreads();
  *total = tot;
  return off + inc - v;
}

// ------------------------------------------------------ 1. pretokenize

// One block per PT_TILE bytes (PT_TILE / 64 start words). Stage the bytes, decode
// every position of the tile and its halo into LDS entries, then each wave
// takes one 64-byte word at a time, lane = byte, and ballots the start bits
// into the word. Positions inside the block are 32-bit offsets from lo (the
// first entry); RS is the ruleset, DM whether document starts are marked.
template <int RS, bool DM>
__global__ __launch_bounds__(PRETOK_TPB) __attribute__((amdgpu_waves_per_eu(7, 7))) void k_pretok(DevTables t, DevWork w,
                                                       int64_t nwords) {
  __shared__ __align__(16) uint8_t sb[PT_BYTES];
  __shared__ uint32_t se[PT_SPAN];
  // the NFC quick-check value of each span position's code point
  __shared__ uint8_t snfc[PT_SPAN];
  __shared__ uint64_t sdm[PT_DMW];
  __shared__ uint64_t sw[PT_TILE / 64 + 1];  // the tile's start words + next
  __shared__ uint32_t lcnt[PACK_CLASSES];
  // pieces over 64 bytes that start in the tile (at most PT_TILE / 65)
  __shared__ uint32_t llong[PT_TILE / 64], nlong, longbase;
  // the first 256 code points' class and NFC value and the 256 byte ids,
  // one 32-bit word per entry (LTAB_*): LDS copies for the common case (one
  // entry per thread; 32-bit words, so the compiler keeps the LDS and HBM
  // table reads apart instead of merging them into one flat load)
  static_assert(PRETOK_TPB == 256, "one table entry per thread");
  __shared__ uint32_t ltab[256];
  // where the tile's pieces of each class go in plist
  __shared__ uint32_t lbase[PACK_CLASSES];
  // digit groups (\p{N}{1,K}, K > 1), per word from the halo word to the
  // first word after the tile: N-class character starts, run breaks (other
  // character starts and document starts), and the N characters of the run
  // at the word's end
  __shared__ uint64_t gNL[PT_TILE / 64 + 2], gBR[PT_TILE / 64 + 2];
  __shared__ uint32_t gC[PT_TILE / 64 + 1];
  // (o200k) the functions of the words before the waves' blocks, the
  // blocks' functions, and the blocks' entry states
  __shared__ uint32_t o2w[4][4], o2b[4][4];
  __shared__ uint32_t o2e[4];
  const int tid = threadIdx.x;
  if (tid < PACK_CLASSES) lcnt[tid] = 0;
  if (tid == 0) nlong = 0;
  {
    const int32_t bid = t.byte_id[tid];
    ltab[tid] = (bid >= 0 ? (uint32_t)bid : LTAB_NOID) |
                ((uint32_t)t.cls[tid] << LTAB_CLS) |
                ((w.check_nfc ? (uint32_t)t.nfc[tid] : 0u) << LTAB_NFC);
  }
  const int64_t base = (int64_t)blockIdx.x * PT_TILE;
  const int64_t nb = w.nb;
  const bool al = ((uintptr_t)w.text & 15) == 0;
  for (int j = tid; j < PT_BYTES / 16; j += PRETOK_TPB) {
    const int64_t p = base - PT_PAD + 16 * j;
    uint4 v;
    if (al && p >= 0 && p + 16 <= nb) {
      v = *reinterpret_cast<const uint4*>(w.text + p);
    } else {
      uint32_t x[4] = {0, 0, 0, 0};
      for (int k = 0; k < 16; ++k) {
        const int64_t q = p + k;
        if (q >= 0 && q < nb) x[k >> 2] |= (uint32_t)w.text[q] << (8 * (k & 3));
      }
      v = make_uint4(x[0], x[1], x[2], x[3]);
    }
    *reinterpret_cast<uint4*>(sb + 16 * j) = v;
  }
  // Clear what the later stages of this call accumulate into: the block's
  // words of the long-piece masks, the words of repair bits whose first
  // covered word is one of the block's (a repair word covers 64 words), and
  // (block 0) the control slot of the next call; the last block takes the
  // tails.
  {
    constexpr int64_t TW = PT_TILE / 64;
    const int64_t wd0 = (base >> 6);
    const int64_t dw0 = (wd0 + 63) / 64, dw1 = (wd0 + TW + 63) / 64;
    const bool last = blockIdx.x == gridDim.x - 1;
    for (int64_t j = wd0 + tid; j < w.clear_words && (j < wd0 + TW || last);
         j += PRETOK_TPB) {
      w.inlong[j] = 0;
      w.failm[j] = 0;
    }
    for (int64_t j = dw0 + tid; j < w.clear_dwords && (j < dw1 || last);
         j += PRETOK_TPB)
      w.dirty_next[j] = 0;
    if (blockIdx.x == 0)
      for (int j = tid; j < CTRL_WORDS; j += PRETOK_TPB) w.ctrl_next[j] = 0;
  }
  const int64_t wlo = (base >> 6) - 3;
  // dm: the staged mask words hold a document start. A block without one
  // decides as if documents were not marked (the same answers: the mask
  // only matters where it has bits, and positions past the staged words go
  // to the mask in HBM either way).
  bool dm = false;
  if (DM) {
    const int64_t nmw = nb / 64 + 2;  // words the caller's mask holds
    int nz = 0;
    for (int j = tid; j < PT_DMW; j += PRETOK_TPB) {
      const int64_t wd = wlo + j;
      const uint64_t v = (wd >= 0 && wd < nmw) ? w.docmask[wd] : 0;
      sdm[j] = v;
      nz |= v != 0;
    }
    dm = __syncthreads_or(nz) != 0;
  } else {
    __syncthreads();
  }
  const int64_t lo = base - PT_HALO;
  // entries within the text: local offsets [jlo, jhi)
  const int jlo = lo < 0 ? (int)(-lo) : 0;
  const int jhi = nb - lo < PT_SPAN ? (int)(nb - lo) : PT_SPAN;
  for (int j = tid; j < PT_SPAN; j += PRETOK_TPB) {
    const int sj = j + (PT_PAD - PT_HALO);  // its byte in sb
    uint32_t e = 0;
    uint8_t snf = 0;
    {
      // the step from this position to the previous character's lead
      // (back of the byte before, with its own position clamp)
      const int64_t pos = lo + j;
      const bool u1 = is_cont(sb[sj - 1]) && pos > 1;
      const bool u2 = u1 && is_cont(sb[sj - 2]) && pos > 2;
      const bool u3 = u2 && is_cont(sb[sj - 3]) && pos > 3;
      e = (uint32_t)(u1 + u2 + u3) << 30;
    }
    if (j >= jlo && j < jhi) {
      const int pg = lo + j < 3 ? (int)(lo + j) : 3;  // min(position, 3)
      const uint32_t b0 = sb[sj], b1 = sb[sj + 1], b2 = sb[sj + 2], b3 = sb[sj + 3];
      const bool c0 = is_cont(b0), c1 = is_cont(b1), c2 = is_cont(b2), c3 = is_cont(b3);
      const bool m1 = is_cont(sb[sj - 1]), m2 = is_cont(sb[sj - 2]);
      const bool m3 = is_cont(sb[sj - 3]);
      // steps back to a lead over at most three continuation bytes (never
      // below position 0); continuation bytes after this one (bytes past
      // the text are staged as 0)
      const int back = (pg > 0 && c0) ? ((pg > 1 && m1) ? ((pg > 2 && m2) ? 3 : 2) : 1) : 0;
      const int fwd = c1 ? (c2 ? (c3 ? 3 : 2) : 1) : 0;
      // UTF-8 decode, valid forms only (U+FFFD otherwise)
      const int n = b0 < 0x80 ? 0 : b0 < 0xC0 ? 4 : b0 < 0xE0 ? 1 : b0 < 0xF0 ? 2 : b0 < 0xF8 ? 3 : 4;
      const int64_t avail = nb - (lo + j);
      const uint32_t v = n == 0 ? b0
                       : n == 1 ? ((b0 & 0x1F) << 6) | (b1 & 0x3F)
                       : n == 2 ? ((b0 & 0x0F) << 12) | ((b1 & 0x3F) << 6) | (b2 & 0x3F)
                       : ((b0 & 0x07) << 18) | ((b1 & 0x3F) << 12) | ((b2 & 0x3F) << 6) | (b3 & 0x3F);
      const bool bad = n == 4 || n >= avail || (n >= 1 && !c1) ||
                       (n >= 2 && !c2) || (n >= 3 && !c3) ||
                       (n == 1 && v < 0x80) || (n == 2 && v < 0x800) ||
                       (n == 3 && v < 0x10000) || v > 0x10FFFF ||
                       (v >= 0xD800 && v <= 0xDFFF);
      const uint32_t cp = bad ? 0xFFFDu : v;
      uint32_t cl, nv;
      if (cp < 256) {
        const uint32_t lt = ltab[cp];
        cl = (lt >> LTAB_CLS) & 7;
        nv = lt >> LTAB_NFC;
      } else {
        cl = t.cls[cp];
        nv = w.check_nfc ? t.nfc[cp] : 0u;
      }
      snf = (uint8_t)nv;
      // a continuation byte is valid when the first byte back that is not
      // one (at most three back, not before position 0) is a lead that
      // announces at least that many continuation bytes
      bool ok = !bad;
      if (c0) {
        const int d = !m1 ? 1 : !m2 ? 2 : !m3 ? 3 : 4;
        const uint32_t l = sb[sj - (d < 4 ? d : 3)];
        const int need = l >= 0xF8 ? 0 : l >= 0xF0 ? 3 : l >= 0xE0 ? 2 : l >= 0xC0 ? 1 : 0;
        ok = d <= pg && need >= d;
      }
      e |= cp | ((cl & 3) << 21) | ((cl >> 2) << 28) | ((uint32_t)back << 23) |
          ((uint32_t)fwd << 25) | (ok ? 1u << 27 : 0u);
    }
    se[j] = e;
    snfc[j] = snf;
  }
  __syncthreads();
  const int lane = tid & 63, wv = wave_id();
  // the ruleset's class of an entry, and its digit / P / whitespace classes
  auto kcl = [](uint32_t e) {
    return RS == RS_DEEPSEEK || RS == RS_O200K || RS == RS_KIMI ? dcl(e) : ecl(e);
  };
  constexpr int KN = RS == RS_DEEPSEEK ? DS_N : RS == RS_O200K || RS == RS_KIMI ? OK_N : CN_;
  constexpr int KP = RS == RS_DEEPSEEK ? DS_PS : CP_;
  auto kws = [](int k) { return RS == RS_DEEPSEEK ? k >= DS_WS : k == CS_; };
  // Digit groups (\p{N}{1,K}, K > 1) count the N characters of the run
  // before a digit, and a run can be any length. Per word of the span from
  // the halo word on, the N-class character starts (gNL) and the run breaks
  // (gBR: the starts of other characters, and document starts, where a run
  // begins), index k + 1 for word k (-1: the halo word, PT_TILE / 64: the
  // first word after the tile, which the start words recompute); thread 0
  // counts the run's N characters at every word end up to the tile's (gC,
  // index k + 1 for tile word k, 0 for the halo word). A run that reaches
  // back past the halo takes its count before the tile from the tiles
  // before: each tile publishes, before it waits on anything, the N
  // characters of the run at its end and whether the run spans it whole,
  // tagged with the call number, and a tile whose halo holds no break reads
  // its predecessors' (bounded waits). Every digit is then one lookup.
  uint32_t st = 0;  // status bits of the tile
  const bool groups = (RS == 0 || RS == RS_DEEPSEEK || RS == RS_O200K) && t.dmax > 1;
  if (groups) {
    for (int k = wv - 1; k <= PT_TILE / 64; k += PRETOK_TPB / 64) {
      const int64_t p = base + 64 * k + lane;
      const int L = PT_HALO + 64 * k + lane;
      const bool ld = p >= 0 && p < nb && !is_cont(sb[L + (PT_PAD - PT_HALO)]);
      const bool isn = ld && kcl(se[L]) == KN;
      bool dsp = p == 0;
      if (DM && dm && ld && !dsp) dsp = (sdm[(p >> 6) - wlo] >> (p & 63)) & 1;
      const uint64_t mn = __ballot(isn);
      const uint64_t mb = __ballot(ld && (!isn || dsp));
      if (lane == 0) {
        gNL[k + 1] = mn;
        gBR[k + 1] = mb;
      }
    }
    __syncthreads();
    if (wv == 0) {
      // Wave 0, lane k for tile word k (1 .. TW): the N characters of the
      // run at the word's end, as a segmented prefix sum (a word with a
      // break restarts the run at its last break; a document start that is
      // an N character opens the run and counts).
      constexpr int TW = PT_TILE / 64;
      static_assert(TW < 64, "a lane per tile word");
      const bool act = lane >= 1 && lane <= TW;
      const uint64_t bw = act ? gBR[lane] : 0, nw = act ? gNL[lane] : 0;
      uint32_t ab = 0;  // N characters after the word's last break
      if (bw) {
        const int h = 63 - __builtin_clzll(bw);
        ab = (uint32_t)__popcll(nw & ~mask_le(h)) + (uint32_t)((nw >> h) & 1);
      }
      const uint32_t P = wave_incl_scan((uint32_t)__popcll(nw), lane);
      const uint64_t bm = __ballot(bw != 0);
      const uint64_t le = bm & mask_le(lane);
      const int lb = le ? 63 - __builtin_clzll(le) : 0;  // the last word with a break
      const uint32_t abl = (uint32_t)__shfl((int)ab, lb);
      const uint32_t Pl = (uint32_t)__shfl((int)P, lb);
      const uint32_t run = le ? abl + (P - Pl) : P;
      if (act) gC[lane] = run;
      // the tile's first word with a break, less one (TW: none)
      const int fb = bm ? __builtin_ctzll(bm) - 1 : TW;
      const uint32_t run_end = (uint32_t)__builtin_amdgcn_readlane((int)run, TW);
      uint32_t c0 = 0;
      if (lane == 0) {
        if (w.nrun)
          nrun_store(&w.nrun[blockIdx.x], ((uint64_t)w.seq << 32) |
                                              (fb == TW ? NRUN_FULL : 0) | run_end);
        if (gBR[0]) {
          const uint64_t b0 = gBR[0], n0 = gNL[0];
          const int h = 63 - __builtin_clzll(b0);
          c0 = (uint32_t)__popcll(n0 & ~mask_le(h)) + (uint32_t)((n0 >> h) & 1);
        } else if (gNL[0] && w.nrun) {
          // the run reaches back past the halo: the tiles before it
          WaitBound wb;
          for (int64_t u = (int64_t)blockIdx.x - 1; u >= 0; --u) {
            uint64_t v;
            while ((uint32_t)((v = nrun_load(&w.nrun[u])) >> 32) != w.seq) {
              if (wb.expired(w.wait_ticks)) break;
              __builtin_amdgcn_s_sleep(2);
            }
            if ((uint32_t)(v >> 32) != w.seq) {
              st |= ST_STALL_PRETOK;
              break;
            }
            c0 += (uint32_t)(v & (NRUN_FULL - 1));
            if (!(v & NRUN_FULL)) break;
          }
        }
        gC[0] = c0;
      }
      c0 = (uint32_t)__shfl((int)c0, 0);
      if (act && lane <= fb) gC[lane] = run + c0;
    }
    __syncthreads();
  }
  const LCtx c{GCtx{w.text, nb, DM ? w.docmask : nullptr, t.cls}, se, lo, sdm, wlo};
  // document start at local offset L: position 0, or a marked doc head
  const int Lz = lo <= 0 ? (int)(-lo) : -1;
  auto prv = [&](int L) {  // local offset of the character before L
    return L - 1 - (int)(se[L] >> 30);
  };
  // the tile's words, and the first word after it (the next block writes
  // that one; it is recomputed here to size the pieces near the tile end)
  // The start words, compiled twice: with document starts in the staged
  // mask words (D) and without (the common case, where none of the
  // document checks is needed); a block takes one of the two.
  auto start_words = [&](auto dflag) {
    constexpr bool D = decltype(dflag)::value;
    // every span position's mask word is staged (words tile - 1 .. tile +
    // PT_TILE / 64 of the PT_DMW from tile - 3), so D reads LDS only
    auto ds = [&](int L) {
      if (!D) return L == Lz;
      const int64_t i = lo + L;
      return i == 0 || ((sdm[(i >> 6) - wlo] >> (i & 63)) & 1) != 0;
    };
    // (deepseek) the highest position <= from that is not an ASCII letter
    // or that opens a document: the staged bytes 64 a step, then the text
    // in HBM (ds_stop_hbm); position 0 opens the text, so the search ends.
    // Wave-uniform, from >= 0.
    auto ds_stop = [&](int64_t from) -> int64_t {
      const int64_t st0 = base - PT_PAD;  // the position of sb[0]
      const int64_t lo_st = st0 > 0 ? st0 : 0;
      for (int64_t top = from; top >= lo_st; top -= 64) {
        const int64_t p = top - lane;
        bool stop = false;
        if (p >= lo_st) stop = !ascii_alpha(sb[p - st0]) || ds((int)(p - lo));
        const uint64_t m = __ballot(stop);
        if (m) return top - __builtin_ctzll(m);
      }
      // (lo_st == 0: position 0 stopped the loop above; guarded all the same)
      return lo_st > 0 ? ds_stop_hbm(w.text, c.g.dm, lo_st - 1) : (int64_t)-1;
    };
    for (int k = wv; k <= PT_TILE / 64; k += PRETOK_TPB / 64) {
      const int64_t wd = (base >> 6) + k;
      if (wd >= nwords) {  // past the sentinel words: all starts
        if (lane == 0) sw[k] = ~0ULL;
        continue;
      }
      const int64_t i = base + 64 * k + lane;
      const int Li = PT_HALO + 64 * k + lane;  // i - lo
      const int sj = 64 * k + lane + PT_PAD;
      // ASCII byte kinds across the word (bytes past the text are 0): the
      // run-level cases below read them instead of walking the run
      const uint32_t bb = sb[sj];
      const uint64_t mWS = __ballot(bb == ' ' || bb == '\t' || bb == 0x0B || bb == 0x0C);
      const uint64_t mCR = __ballot(bb == '\n' || bb == '\r');
      const uint64_t mHI = __ballot(bb >= 0x80);
      // (deepseek) ASCII letters, for [ascii punct][A-Za-z]+ runs
      const uint64_t mAL = RS == RS_DEEPSEEK ? __ballot(ascii_alpha((int)bb)) : 0ULL;
      // Every lane evaluates the fast predicate from the fixed context (only
      // selects); the lanes it leaves open (runs to walk, the general path)
      // are resolved in a section the wave enters only when it has any.
      const bool in = i < nb;
      const bool lead = in && !is_cont((uint8_t)bb);
      // the entry's valid bit: a lead that decodes, or a continuation byte
      // that a lead claims
      const uint32_t e = se[Li];
      if (in && !((e >> 27) & 1)) st |= ST_UTF8;
      const bool d0 = ds(Li);
      // the fixed context: every offset used lies in the LDS span (tile
      // positions are at least PT_HALO from either end, and the four
      // characters back cover at most 16 bytes); the one after is checked
      // (each step back reads one entry: the entry holds the step to the
      // character before it; the steps past a document start are read all
      // the same and not used, h2 .. h4)
      Ctx5 x;
      x.c0 = e;
      const int L1 = Li - 1 - (int)(e >> 30);
      x.c1 = se[L1];
      const int L2 = L1 - 1 - (int)(x.c1 >> 30);
      x.c2 = se[L2];
      const int L3 = L2 - 1 - (int)(x.c2 >> 30);
      x.c3 = se[L3];
      const int L4 = L3 - 1 - (int)(x.c3 >> 30);
      x.c4 = se[L4];
      x.h2 = !ds(L1);
      x.h3 = x.h2 && !ds(L2);
      x.h4 = x.h3 && !ds(L3);
      const int Ln = Li + 1 + (int)((e >> 25) & 3);
      const bool nin = Ln < PT_SPAN;
      x.hn = lo + Ln < nb && !ds(Ln);
      x.cn = nin ? se[Ln] : 0u;
      int r = !nin ? -1
            : RS == 1 ? fast_r50k(x)
            : RS == RS_DEEPSEEK ? fast_deepseek(x, t.dmax)
                                : fast_cl100k(x, t.dmax);
      // a digit's group needs nothing after it: the run count decides
      // (also at the span's last byte, where the fixed context stops)
      if (groups && kcl(e) == KN) r = FAST_DIGITS;
      const bool open = lead && !d0 && r < 0;
      int64_t far = -1;  // (deepseek) FAST_FAR: where the search starts
      if (__builtin_amdgcn_ballot_w64(open)) {  // wave-uniform
        if (open) {
          const uint64_t below = (1ULL << lane) - 1;
          // document starts in this word (a run ends at one, as at the
          // text end)
          const uint64_t dmw = D ? sdm[wd - wlo] : 0;
          if (r == FAST_DIGITS) {
            // the N characters of the run before i: after the last break
            // below it in the word, else the count at the previous word's
            // end plus the word's N characters below it
            const uint64_t n = gNL[k + 1], b = gBR[k + 1] & below;
            uint32_t cnt;
            if (b) {
              const int h = 63 - __builtin_clzll(b);
              cnt = (uint32_t)__popcll(n & below & ~mask_le(h)) + (uint32_t)((n >> h) & 1);
            } else {
              cnt = gC[k] + (uint32_t)__popcll(n & below);
            }
            r = cnt % (uint32_t)t.dmax == 0;
          } else if (r == FAST_CRLF && bb < 0x80) {
            // another CR/LF ahead in the run: it shows in the word before
            // the first byte that is neither (unless that byte is not
            // ASCII) and before the next document start
            const uint64_t above = ~mask_le(lane);
            const uint64_t stop = ~(mWS | mCR) & above;
            const int f = stop ? __builtin_ctzll(stop) : 64;
            const int fd = (dmw & above) ? __builtin_ctzll(dmw & above) : 64;
            const int g = (mCR & above) ? __builtin_ctzll(mCR & above) : 64;
            if (g < f && g < fd) {
              // then the char before the CR/LF run that precedes i (none
              // when a document starts inside that run)
              const uint64_t nc = ~mCR & below;
              const int h = nc ? 63 - __builtin_clzll(nc) : -1;
              if (dmw & lanes_in(h + 1, lane)) {
                r = 0;
              } else if (h >= 0) {
                if ((mWS >> h) & 1) r = 0;
                else if (!((mHI >> h) & 1)) r = kcl(se[Li - (lane - h)]) == KP;
              }
            } else if (fd < 64 && fd <= f) {
              r = 1;
            } else if (f < 64 && !((mHI >> f) & 1)) {
              r = 1;
            }
          } else if (RS == RS_DEEPSEEK && r == FAST_GENERAL) {
            // a letter / mark after an ASCII-alpha run longer than the
            // context (ds_run_led): the highest byte below the lane that is
            // not an ASCII letter or that opens a document decides; when
            // the run reaches back past the word's first byte the wave
            // searches for it below (FAST_FAR)
            const uint64_t stop = (~mAL | dmw | (wd == 0 ? 1ULL : 0ULL)) & below;
            if (stop) {
              r = ds_run_led(c, i - (lane - (63 - __builtin_clzll(stop))));
            } else {
              r = FAST_FAR;
              far = i - lane - 1;
            }
          }
          if (r == FAST_CRLF) {
            // end of \s*[\r\n]+ unless another CR/LF follows in the run;
            // then the first char the P match's [\r\n]* left over
            r = -1;
            bool more = false, known = false;
            for (int L = Ln;;) {
              if (lo + L >= nb || ds(L)) { known = true; break; }
              if (L >= PT_SPAN) break;
              const uint32_t eq = se[L];
              if (!kws(kcl(eq))) { known = true; break; }
              if (crlf(ecp(eq))) { more = known = true; break; }
              L += 1 + (int)((eq >> 25) & 3);
            }
            if (known && !more) r = 1;
            if (known && more) {
              for (int L = L1;;) {
                if (ds(L)) { r = 0; break; }
                if (L - 1 < 0) break;
                const int Lr = prv(L);
                const uint32_t ex = se[Lr];
                // (a DeepSeek P/S character of a CJK run is another region:
                // the CR/LF run starts its own)
                if (!kws(kcl(ex))) {
                  r = kcl(ex) == KP && !(RS == RS_DEEPSEEK && ds_cjk(ecp(ex)));
                  break;
                }
                if (!crlf(ecp(ex))) { r = 0; break; }
                L = Lr;
              }
            }
          }
          if (r < 0 && r != FAST_FAR) {
            const Ch ci{i, (int32_t)(e & 0x1FFFFF), (uint8_t)kcl(e)};
            r = RS == 1 ? start_r50k(c, ci)
              : RS == RS_DEEPSEEK ? start_deepseek(c, ci, t.dmax, &far)
                                  : start_cl100k(c, ci, t.dmax);
          }
        }
        if (RS == RS_DEEPSEEK) {
          // the ASCII-alpha runs that reach below the word (at most one a
          // word, the word's first run) or the span: one search each by
          // the whole wave, with no wait on another tile
          uint64_t farm = __ballot(open && r == FAST_FAR);
          while (farm) {
            const int l = __builtin_ctzll(farm);
            farm &= farm - 1;
            const int64_t from = ((int64_t)__builtin_amdgcn_readlane((int)(far >> 32), l) << 32) |
                                 (uint32_t)__builtin_amdgcn_readlane((int)far, l);
            const int64_t s = ds_stop(from);
            if (lane == l) r = ds_run_led(c, s);
          }
        }
      }
      // sentinel starts past the text; no start inside a character
      const bool s = !in || (lead && (d0 || r != 0));
      if (w.check_nfc && lead) {
        const uint32_t v = snfc[Li];
        if (v == 255 || (v != 0 && !d0 && snfc[L1] > v)) st |= ST_NFC;
      }
      uint64_t m = __ballot(s);
      // no start inside an added-token literal (its first byte is a document
      // start already)
      if (DM && w.litb) m &= ~w.litb[wd];
      if (lane == 0) {
        sw[k] = m;
        if (k < PT_TILE / 64) w.starts[wd] = m;
      }
    }
  };
  // o200k / kimi: the automaton over the tile (o2k_char). Wave wv takes the
  // contiguous words [12 wv, 12 wv + 12) (wave 3 also the word after the
  // tile) and carries the state from word to word. Its entry state is the
  // function of the word before its block when that function is constant
  // (on ordinary text it is). Otherwise every wave first composes its
  // block's function, and thread 0 takes the tile's entry from the word
  // before the tile or from the tiles before it (each tile publishes its
  // whole function before it looks back, and the state after it once
  // known: a decoupled look-back with bounded waits) and derives the
  // blocks' entries. Every tile publishes the state after it.
  auto o2k_words = [&](auto dflag) {
    constexpr bool D = decltype(dflag)::value;
    auto ds = [&](int L) {
      if (!D) return L == Lz;
      const int64_t i = lo + L;
      return i == 0 || ((sdm[(i >> 6) - wlo] >> (i & 63)) & 1) != 0;
    };
    constexpr int WPB = PT_TILE / 64 / (PRETOK_TPB / 64);  // words per wave
    constexpr int NST = o2_nst<RS>();
    constexpr int W = o2_words<RS>();
    using Fn = O2Fn<W>;
    constexpr uint32_t ALL = (1u << NST) - 1;
    const bool contr = t.contractions != 0;
    // the lane's transition and start bits in word k (-1 .. PT_TILE / 64);
    // positions outside the text and inside a character pass the state on
    auto lane_fn = [&](int k, bool need_g, Fn* f, uint32_t* g) {
      const int64_t i = base + 64 * k + lane;
      const int Li = PT_HALO + 64 * k + lane;
      const uint32_t bb = sb[64 * k + lane + PT_PAD];
      // ASCII whitespace, CR/LF and non-ASCII bytes across the word (bytes
      // past the text are staged as 0): a whitespace character after a
      // CR/LF reads whether another CR/LF follows in its run from them
      int ws_hint = -1;
      if (need_g) {
        const uint64_t mWS = __ballot(bb == ' ' || bb == '\t' || bb == 0x0B || bb == 0x0C);
        const uint64_t mCR = __ballot(bb == '\n' || bb == '\r');
        const uint64_t mHI = __ballot(bb >= 0x80);
        const uint64_t above = ~mask_le(lane);
        const uint64_t stop = ~(mWS | mCR) & above;
        const int fs = stop ? __builtin_ctzll(stop) : 64;
        const uint64_t dmw = D ? sdm[(base >> 6) + k - wlo] & above : 0;
        const int fd = dmw ? __builtin_ctzll(dmw) : 64;
        const int gc = (mCR & above) ? __builtin_ctzll(mCR & above) : 64;
        const int end = fd < fs ? fd : fs;  // the run's end, as far as the masks go
        if (gc < end) ws_hint = 0;
        else if (fd <= fs && fd < 64) ws_hint = 1;
        else if (fs < 64 && !((mHI >> fs) & 1)) ws_hint = 1;
      }
      *f = o2_ident<W>();
      *g = 0;
      if (i < 0 || i >= nb || is_cont((uint8_t)bb)) return;
      const uint32_t e = se[Li];
      const int kc = dcl(e);
      const bool d0 = ds(Li);
      // the characters before and after it (from the staged entries; the
      // first lanes of the halo word and the last of the word after the
      // tile read the text)
      uint32_t xp = 0, x1 = 0;
      bool hp = false, h1 = false;
      if (!d0) {
        if (Li >= 4) {
          const int Lp = prv(Li);
          xp = se[Lp];
          hp = true;
        } else {
          const int64_t q = c.prev(i);
          if (q >= 0) {
            const Ch x = c.at(q);
            xp = (uint32_t)x.cp | ((uint32_t)(x.cl & 3) << 21) | ((uint32_t)(x.cl >> 2) << 28);
            hp = true;
          }
        }
      }
      const int Ln = Li + 1 + (int)((e >> 25) & 3);
      if (Ln < PT_SPAN) {
        h1 = lo + Ln < nb && !ds(Ln);
        if (h1) x1 = se[Ln];
      } else {
        const int64_t q = c.next(i);
        if (q >= 0) {
          const Ch x = c.at(q);
          x1 = (uint32_t)x.cp | ((uint32_t)(x.cl & 3) << 21) | ((uint32_t)(x.cl >> 2) << 28);
          h1 = true;
        }
      }
      o2k_char<RS>(c, i, e, d0, xp, hp, x1, h1, need_g, contr, ws_hint, f, g);
      if (RS == RS_O200K && need_g && kc == OK_N && !d0) {
        // \p{N}{1,K}: the N characters of the run before i decide
        bool r = true;
        if (groups) {
          const uint64_t below = (1ULL << lane) - 1;
          const uint64_t n = gNL[k + 1], b = gBR[k + 1] & below;
          uint32_t cnt;
          if (b) {
            const int h = 63 - __builtin_clzll(b);
            cnt = (uint32_t)__popcll(n & below & ~mask_le(h)) + (uint32_t)((n >> h) & 1);
          } else {
            cnt = gC[k] + (uint32_t)__popcll(n & below);
          }
          r = cnt % (uint32_t)t.dmax == 0;
        }
        *g = r ? ALL : 0u;
      }
    };
    // the function of word k (lane 63's composition), wave-uniform
    auto word_fn = [&](int k) {
      Fn f;
      uint32_t g;
      lane_fn(k, false, &f, &g);
      return o2_lane63(o2_scan(f));
    };
    // word k from entry state `carry`: its start word; returns the state
    // after it
    auto word = [&](int k, uint32_t carry) -> uint32_t {
      const int64_t wd = (base >> 6) + k;
      if (wd >= nwords) {  // past the sentinel words: all starts
        if (lane == 0) sw[k] = ~0ULL;
        return carry;
      }
      Fn f;
      uint32_t g;
      lane_fn(k, true, &f, &g);
      const uint32_t sj = o2_at(o2_scan(f), carry);  // the state after the lane
      // the state before it: the lane before's (wave_shr:1), carry at lane 0
      const uint32_t sp = (uint32_t)__builtin_amdgcn_update_dpp((int)carry, (int)sj, 0x138,
                                                                0xF, 0xF, false);
      const int64_t i = base + 64 * k + lane;
      const int Li = PT_HALO + 64 * k + lane;
      const uint32_t bb = sb[64 * k + lane + PT_PAD];
      const bool in = i < nb;
      const bool lead = in && !is_cont((uint8_t)bb);
      const uint32_t e = se[Li];
      if (in && !((e >> 27) & 1)) st |= ST_UTF8;
      // sentinel starts past the text; no start inside a character
      const bool s = !in || (lead && ((g >> sp) & 1));
      if (w.check_nfc && lead) {
        const uint32_t v = snfc[Li];
        if (v == 255 || (v != 0 && !ds(Li) && snfc[prv(Li)] > v)) st |= ST_NFC;
      }
      uint64_t m = __ballot(s);
      if (DM && w.litb) m &= ~w.litb[wd];
      if (lane == 0) {
        sw[k] = m;
        if (k < PT_TILE / 64) w.starts[wd] = m;
      }
      return (uint32_t)__builtin_amdgcn_readlane((int)sj, 63);
    };
    const int k0 = WPB * wv;
    // the word before the block (the tile's halo word for wave 0); the
    // first tile starts at a document start, whatever came before
    Fn T = word_fn(k0 - 1);
    if (blockIdx.x == 0 && wv == 0) T = o2_rep<W>(O2_FRESH);
    if (lane == 0)
      for (int q = 0; q < W; ++q) o2w[wv][q] = T.d[q];
    __syncthreads();
    auto lds_fn = [&](const uint32_t (*a)[4], int j) {
      Fn f;
#pragma unroll
      for (int q = 0; q < W; ++q) f.d[q] = a[j][q];
      return f;
    };
    bool fast = true;
    for (int j = 0; j < PRETOK_TPB / 64; ++j) fast &= o2_const<RS>(lds_fn(o2w, j));
    uint32_t carry;
    uint64_t* op = w.ostate + 2 * (int64_t)blockIdx.x;
    if (fast) {
      carry = o2w[wv][0] & 0xFFu;
    } else {
      Fn B = o2_ident<W>();
      for (int k = k0; k < k0 + WPB; ++k) B = o2_then(B, word_fn(k));
      if (lane == 0)
        for (int q = 0; q < W; ++q) o2b[wv][q] = B.d[q];
      __syncthreads();
      if (tid == 0) {
        Fn A = lds_fn(o2b, 0);
        for (int j = 1; j < PRETOK_TPB / 64; ++j) A = o2_then(A, lds_fn(o2b, j));
        uint32_t entry = O2_FRESH;
        const Fn H = lds_fn(o2w, 0);
        if (o2_const<RS>(H)) {
          entry = o2_at(H, 0);
        } else {
          o2_publish(op, w.seq, O2_AGG, o2_pack<RS>(A), 0);
          // G: the function of the tiles after u up to this one
          Fn G = o2_ident<W>();
          bool done = false;
          WaitBound wb;
          for (int64_t u = (int64_t)blockIdx.x - 1; u >= 0 && !done; --u) {
            const uint64_t* q = w.ostate + 2 * u;
            uint64_t v1;
            while ((uint32_t)((v1 = __hip_atomic_load(q + 1, __ATOMIC_ACQUIRE,
                                                      __HIP_MEMORY_SCOPE_AGENT)) >> 32) !=
                   w.seq) {
              if (wb.expired(w.wait_ticks)) break;
              __builtin_amdgcn_s_sleep(2);
            }
            if ((uint32_t)(v1 >> 32) != w.seq) {
              st |= ST_STALL_PRETOK;
              done = true;
            } else if (((v1 >> 30) & 3) == O2_INCL) {
              entry = o2_at(G, (uint32_t)(v1 >> 26) & 15);
              done = true;
            } else {
              const uint64_t v0 = __hip_atomic_load(q, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
              G = o2_then(o2_unpack<RS>((uint32_t)v0 | ((v1 & 0xFFFFF) << 32)), G);
              if (o2_const<RS>(G)) {
                entry = o2_at(G, 0);
                done = true;
              }
            }
          }
          // (past tile 0 nothing came before: position 0 starts a document)
          if (!done) entry = o2_at(G, O2_FRESH);
        }
        o2_publish(op, w.seq, O2_INCL, 0, o2_at(A, entry));
        o2e[0] = entry;
        for (int j = 1; j < PRETOK_TPB / 64; ++j) o2e[j] = o2_at(lds_fn(o2b, j - 1), o2e[j - 1]);
      }
      __syncthreads();
      carry = o2e[wv];
    }
    for (int k = k0; k < k0 + WPB; ++k) carry = word(k, carry);
    if (wv == PRETOK_TPB / 64 - 1) {
      if (fast && lane == 0) o2_publish(op, w.seq, O2_INCL, 0, carry);
      word(PT_TILE / 64, carry);
    }
  };
  if constexpr (RS == RS_O200K || RS == RS_KIMI) {
    if (DM && dm) o2k_words(std::true_type{});
    else o2k_words(std::false_type{});
  } else {
    if (DM && dm) start_words(std::true_type{});
    else start_words(std::false_type{});
  }
  if (st) atomicOr(w.status, st);
  __syncthreads();
  // Stage-2 bookkeeping for the pieces that start in this tile: finish the
  // one- and two-byte ones, queue the long ones, and list the rest by class.
  // se (free from here) takes, per position, 0 or the listed piece's class
  // + 1 and index among the tile's pieces of that class; the tile then takes
  // room in its segment's class lists, one counter update per class, and
  // writes the positions there.
  const bool two = !t.ignore_merges;
  for (int k = wv; k < PT_TILE / 64; k += PRETOK_TPB / 64) {
    const int64_t a = base + 64 * k + lane;
    if (a >= nb) break;  // (positions only grow along the loop)
    int kind = piece_kind(sw[k], sw[k + 1], lane, two);
    // a literal's piece is done: its id is in tok already
    if (DM && w.lits && ((w.lits[(base >> 6) + k] >> lane) & 1)) kind = PIECE_NONE;
    uint32_t tag = 0;
    if (kind >= 0) {
      tag = (uint32_t)(kind + 1) | atomicAdd(&lcnt[kind], 1u) << 4;
    } else if (kind == PIECE_ONE) {
      const uint32_t id = ltab[sb[64 * k + lane + PT_PAD]] & LTAB_NOID;
      w.tok[a] = id != LTAB_NOID ? id : INVALID_ID;
    } else if (kind == PIECE_TWO) {
      const uint32_t b0 = sb[64 * k + lane + PT_PAD];
      const uint32_t b1 = sb[64 * k + lane + PT_PAD + 1];
      const uint32_t i0 = ltab[b0] & LTAB_NOID, i1 = ltab[b1] & LTAB_NOID;
      const bool h0 = i0 != LTAB_NOID, h1 = i1 != LTAB_NOID;
      const uint64_t mg = (h0 && h1) ? t.bytepair[(b0 << 8) | b1] : ~0ULL;
      w.tok[a] = mg != ~0ULL ? (uint32_t)mg : h0 ? i0 : INVALID_ID;
      w.tok[a + 1] = (mg == ~0ULL && h1) ? i1 : INVALID_ID;
    } else if (kind == PIECE_LONG) {
      llong[atomicAdd(&nlong, 1u)] = (uint32_t)a;
    }
    se[64 * k + lane] = tag;
  }
  __syncthreads();
  // (the long pieces take their room in the queue with one counter update
  // per tile too; their ends are filled in by k_bpe_pack's first waves
  // once every start word is known)
  if (tid < PACK_CLASSES && lcnt[tid]) {
    const int x = blockIdx.x % PACK_XCDS;
    lbase[tid] = pack_seg_list(gridDim.x, x, PACK_LOCAL_OFF[tid]) +
                 atomicAdd(&w.pseg[x * CTRL_PSEG_STRIDE + CTRL_PSEG_COUNT + tid],
                           lcnt[tid]);
  } else if (tid == 64 && nlong) {
    longbase = atomicAdd(w.longcount, nlong);
  }
  __syncthreads();
  {
    const int nt = nb - base < PT_TILE ? (int)(nb - base) : PT_TILE;
    for (int i = tid; i < nt; i += PRETOK_TPB) {
      const uint32_t e = se[i];
      if (e) w.plist[lbase[(e & 15) - 1] + (e >> 4)] = (uint32_t)(base + i);
    }
  }
  if (nlong) {
    for (uint32_t j = tid; j < nlong; j += PRETOK_TPB) {
      const uint32_t k = longbase + j;
      if (k < w.long_cap) {
        w.longlist[2 * k] = llong[j];
        w.longlist[2 * k + 1] = 0;
      } else {
        atomicOr(w.status, ST_LONGOVF);
      }
    }
  }
}

// Launch, optionally with timing events taken from the dispatch itself
// (hipExtLaunchKernel): no marker packets between the stages.
template <typename... KArgs, typename... Args>
void launch_ev(void (*k)(KArgs...), dim3 grid, dim3 block, hipStream_t s,
               hipEvent_t start, hipEvent_t stop, Args... args) {
  if (start || stop)
    hipExtLaunchKernelGGL(k, grid, block, 0, s, start, stop, 0, args...);
  else
    hipLaunchKernelGGL(k, grid, block, 0, s, args...);
}

hipError_t launch_pretok(const DevTables& t, const DevWork& w, hipStream_t s,
                         hipEvent_t start, hipEvent_t stop) {
  const int64_t nwords = (w.nb + 63) / 64 + 2;  // words 0..nwin+1
  const dim3 g((uint32_t)pretok_tiles(w.nb)), b(PRETOK_TPB);
  const bool dm = w.docmask != nullptr;
  if (t.ruleset == 1) {
    if (dm) launch_ev(k_pretok<1, true>, g, b, s, start, stop, t, w, nwords);
    else launch_ev(k_pretok<1, false>, g, b, s, start, stop, t, w, nwords);
  } else if (t.ruleset == RS_DEEPSEEK) {
    if (dm) launch_ev(k_pretok<RS_DEEPSEEK, true>, g, b, s, start, stop, t, w, nwords);
    else launch_ev(k_pretok<RS_DEEPSEEK, false>, g, b, s, start, stop, t, w, nwords);
  } else if (t.ruleset == RS_O200K) {
    if (dm) launch_ev(k_pretok<RS_O200K, true>, g, b, s, start, stop, t, w, nwords);
    else launch_ev(k_pretok<RS_O200K, false>, g, b, s, start, stop, t, w, nwords);
  } else if (t.ruleset == RS_KIMI) {
    if (dm) launch_ev(k_pretok<RS_KIMI, true>, g, b, s, start, stop, t, w, nwords);
    else launch_ev(k_pretok<RS_KIMI, false>, g, b, s, start, stop, t, w, nwords);
  } else {
    if (dm) launch_ev(k_pretok<0, true>, g, b, s, start, stop, t, w, nwords);
    else launch_ev(k_pretok<0, false>, g, b, s, start, stop, t, w, nwords);
  }
  return hipGetLastError();
}

// ------------------------------------------------ 2. short-piece BPE


// One step of a segmented prefix minimum over the wave: every lane takes the
// minimum with the lane the DPP control names (row_shr:d reads lane - d in
// its row of 16; row_bcast:15 / :31 read lane 15 / 31 into the later rows
// row_mask selects); lanes without a source keep their value.
template <int ctrl, int row_mask>
__device__ __forceinline__ uint32_t dpp_min(uint32_t m) {
  return min(m, (uint32_t)__builtin_amdgcn_update_dpp((int)RANK_INF, (int)m, ctrl,
                                                      row_mask, 0xF, false));
}

// the calling lane's bit of a wave-uniform mask, as a lane predicate
__device__ __forceinline__ bool lane_bit(uint64_t mask) {
  return __builtin_amdgcn_inverse_ballot_w64(mask);
}

constexpr uint32_t SYM_ID = 0xFFFFF;      // token id bits of a packed symbol
constexpr uint32_t SYM_BYTE = 1u << 28;   // the symbol is still one raw byte

// Byte-level BPE of every eligible segment held by one wave; lane holds
// the byte at pos, a segment's bytes sit on consecutive lanes; ps/pe: the
// lane's segment as lanes [ps, pe) (a grid window has pos = base + lane;
// histories are indexed from base + ps, so hist needs that layout). Each round
// every segment merges its lowest-ranked pair (leftmost on equal rank) -- the
// HF order -- until no pair has a rule.
//   vocab_first: a whole piece that is a vocabulary entry is that one
//     token (ignore_merges families; pieces only, never sub-segments).
//   hist: record the merge events that change the segment's first token
//     (hfirst[seg_start + k]) and its last token (hlast[seg_start + k]) as
//     rank<<32|new_id, with the counts in hmeta[seg_start].
//   write: store the ids (token id at its first byte, INVALID_ID at the
//     other bytes of the segment) into tok.
// Returns the final mask of lanes that start a token.
template <bool vocab_first, bool hist, bool write>
__device__ uint64_t wave_bpe(const DevTables& t, const DevWork& w,
                             int64_t base, int64_t pos, int lane, bool elig,
                             int ps, int pe) {
  const uint32_t byte = elig ? w.text[pos] : 0u;
  const int32_t bid = elig ? t.byte_id[byte] : -1;
  uint64_t live = __ballot(bid >= 0);
  if (!__any(elig)) return 0;
  // The lane's symbol in one word for a single cross-lane read: token id
  // (ids fit 20 bits in every table), the raw byte, and SYM_BYTE while the
  // symbol is still that one byte.
  uint32_t sym = (uint32_t)bid | (byte << 20) | SYM_BYTE;
  const int src_ps = ps >= 0 ? ps : lane;

  if (vocab_first && t.ignore_merges) {
    // whole-piece vocabulary hit first (pretok_kernel.cu:921-943 role)
    const bool lead = elig && lane == ps;
    int32_t hit = -1;
    if (lead) hit = vocab_lookup(t, w.text + pos, pe - ps);
    const uint64_t hm = __ballot(hit >= 0);
    const int32_t hid = __shfl(hit, src_ps);
    const bool phit = elig && ((hm >> src_ps) & 1);
    if (phit && lane == ps) sym = (uint32_t)hid;
    live &= ~__ballot(phit && lane != ps);
  }

  // Segment geometry, fixed for the call: the first and last lane of every
  // segment, bit-reversed for the carry chains below. A pair's key is
  // (63 - segment start) << 26 | rank << 6 | lane (ranks < 2^20 - 1): keys
  // of earlier segments are larger, so a wave-wide prefix minimum is each
  // segment's own, and a segment's lowest key -- lowest rank, leftmost on
  // ties -- is the last lane whose key equals its prefix minimum.
  const uint64_t rstarts = __brevll(__ballot(lane == ps));
  const uint64_t ends = __ballot(ps >= 0 && lane == pe - 1);
  const uint64_t rends = __brevll(ends);
  const uint32_t seg_lane = ((uint32_t)(63 - src_ps) << 26) | (uint32_t)lane;
  const uint64_t above = ~mask_le(lane);

  // the lane's pair key (seg_lane | rank << 6) and product; RANK_INF when
  // the lane has no pair with a rule or is no longer live
  uint32_t kx = RANK_INF, mid = 0;
  uint32_t nfirst = 0, nlast = 0;  // event counts, kept by lane ps
  uint64_t dirty = ~0ULL;          // lanes whose pair changed
  for (;;) {
    const uint64_t after = live & above;
    const int nx = after ? __builtin_ctzll(after) : 64;
    // (nx = 64 reads lane 0; that value is never used)
    const uint32_t nsym = (uint32_t)__builtin_amdgcn_ds_bpermute(nx << 2, (int)sym);
    if (lane_bit(dirty)) {
      kx = RANK_INF;
      if (lane_bit(live) && nx < pe) {
        if (sym & nsym & SYM_BYTE) {
          const uint64_t v =
              t.bytepair[((sym >> 12) & 0xFF00) | ((nsym >> 20) & 0xFF)];
          if (v != ~0ULL) { kx = seg_lane | ((uint32_t)(v >> 32) << 6); mid = (uint32_t)v; }
        } else if (t.ctab) {
          uint32_t r_, m_;
          if (ctab_find(t, sym & SYM_ID, nsym & SYM_ID, &r_, &m_)) {
            kx = seg_lane | (r_ << 6);
            mid = m_;
          }
        } else {
          const uint64_t v = pair_lookup(t, sym & SYM_ID, nsym & SYM_ID);
          if (v != ~0ULL) { kx = seg_lane | ((uint32_t)(v >> 32) << 6); mid = (uint32_t)v; }
        }
      }
    }
    const uint32_t key = kx;
    uint32_t m = key;
    m = dpp_min<0x111, 0xF>(m);  // row_shr:1
    m = dpp_min<0x112, 0xF>(m);  // row_shr:2
    m = dpp_min<0x114, 0xF>(m);  // row_shr:4
    m = dpp_min<0x118, 0xF>(m);  // row_shr:8
    m = dpp_min<0x142, 0xA>(m);  // row_bcast:15 into rows 1 and 3
    m = dpp_min<0x143, 0xC>(m);  // row_bcast:31 into rows 2 and 3
    const uint64_t rec = __builtin_amdgcn_ballot_w64(m == key) &
                         ~__builtin_amdgcn_ballot_w64(key == RANK_INF);
    if (rec == 0) break;
    // Each segment's winner is its last record: on the bit-reversed masks a
    // carry started at each segment's last lane runs over the lanes that
    // are neither records nor the segment's first lane and stops on the
    // first that is.
    const uint64_t rrec = __brevll(rec);
    const uint64_t stop = rrec | rstarts;
    const uint64_t wm = __brevll(((~stop + rends) & stop) & rrec);
    const bool win_ = lane_bit(wm);
    if (hist && t.cert == 2) {
      // every merge of the segment, in order (one per round here)
      const uint32_t nr = __shfl(nfirst, src_ps);
      if (win_) {
        const bool lastev = nx + 1 >= pe || ((live & lanes_in(nx + 1, pe)) == 0);
        w.hfirst[base + ps + nr] =
            ((uint64_t)((kx >> 6) & 0xFFFFFu) << 32) |
            (lane == ps ? HR_FIRST : 0) | (lastev ? HR_LAST : 0) | mid;
      }
      if (elig && lane == ps && (wm & lanes_in(ps, pe))) ++nfirst;
    } else if (hist) {
      const uint32_t nf = __shfl(nfirst, src_ps);
      const uint32_t nl = __shfl(nlast, src_ps);
      bool lastev = false;
      if (win_) {
        // the merged pair's right symbol is the segment's last symbol
        lastev = nx + 1 >= pe || ((live & lanes_in(nx + 1, pe)) == 0);
        const uint64_t ev = ((uint64_t)((kx >> 6) & 0xFFFFFu) << 32) | mid;
        if (lane == ps) w.hfirst[base + ps + nf] = ev;
        if (lastev) w.hlast[base + ps + nl] = ev;
      }
      const uint64_t lm = __ballot(lastev);
      if (elig && lane == ps) {
        if (win_) ++nfirst;
        if (lm & lanes_in(ps, pe)) ++nlast;
      }
    }
    // Each winner absorbs the next live lane: a carry from the lane above
    // the winner runs over the dead lanes and lands on it. The same on the
    // bit-reversed masks finds the live lane before each winner, whose
    // right neighbour changed.
    const uint64_t gone = (~live + (wm << 1)) & live;
    if (win_) sym = mid;
    if (lane_bit(gone)) kx = RANK_INF;
    live &= ~gone;
    const uint64_t lr = __brevll(live);
    const uint64_t prevw = __brevll((~lr + (__brevll(wm) << 1)) & lr);
    dirty = wm | prevw;
  }
  if (hist && elig && lane == ps)
    w.hmeta[base + ps] = t.cert == 2 ? nfirst : nfirst | (nlast << 16);
  if (write && elig) w.tok[pos] = lane_bit(live) ? (sym & SYM_ID) : INVALID_ID;
  return live;
}

// Find the end of the segment that starts at `a` and runs past the word
// boundary at 64*wd (bit 0 of word wd is known clear). seg(word) gives the
// boundary bits; the sentinel start bits at and after nb end the search.
template <class SegBits>
__device__ __forceinline__ int64_t seg_end_after(int64_t wd, SegBits seg) {
  uint64_t word = seg(wd);
  while (word == 0) word = seg(++wd);
  return wd * 64 + __builtin_ctzll(word);
}

__device__ __forceinline__ bool fits_a_grid(int64_t a, int64_t b) {
  return b - a <= 64 &&
         (((a >> 6) == ((b - 1) >> 6)) || (((a + 32) >> 6) == ((b - 1 + 32) >> 6)));
}

// Window geometry shared by the grid kernels: phase 0 is the aligned
// window [64v, 64v+64), phase 1 the shifted window [64v-32, 64v+32).
// Given a function word -> boundary bits, returns the window's boundary
// mask S and whether a boundary sits at the window end (E).
template <class SegBits>
__device__ __forceinline__ void window_bits(int64_t v, int phase, SegBits seg,
                                            uint64_t* S, bool* E) {
  if (phase == 0) {
    *S = seg(v);
    *E = seg(v + 1) & 1;
  } else {
    const uint64_t lo = v > 0 ? seg(v - 1) : ~0ULL;
    const uint64_t hi = seg(v);
    *S = (lo >> 32) | (hi << 32);
    *E = (hi >> 32) & 1;
  }
}

// ---- pieces of up to 64 bytes, packed by length
//
// k_pretok listed the pieces by length class (pieces of
// pack_lmin(c)..pack_slot(c) bytes), and k_bpe_pack merges them with one
// wave per work unit of one class. The rounds a wave runs then follow its
// own pieces' lengths rather than the longest piece of a stretch of text.

// end of the piece that starts at a (the next start bit; sentinel bits at
// and past nb end the search)
__device__ __forceinline__ int64_t piece_end(const DevWork& w, int64_t a) {
  const int64_t wd = a >> 6;
  const uint64_t gt = w.starts[wd] & ~mask_le((int)(a & 63));
  if (gt) return wd * 64 + __builtin_ctzll(gt);
  return seg_end_after(wd + 1, [&](int64_t x) { return w.starts[x]; });
}

// the pair's rule as (rank, product id): the compact table when the engine
// built one, else the boundary table
__device__ __forceinline__ bool pair_find(const DevTables& t, uint32_t l,
                                          uint32_t r, uint32_t* rank,
                                          uint32_t* id) {
  if (t.ctab) return ctab_find(t, l, r, rank, id);
  const uint64_t v = pair_lookup(t, l, r);
  *rank = (uint32_t)(v >> 32);
  *id = (uint32_t)v;
  return v != ~0ULL;
}

// One piece of n <= L bytes per lane (n == 0: none), merged serially by its
// lane in the HF order: the lowest-ranked pair, leftmost on ties, one merge
// per step. Positions keep their byte offsets: a live mask per lane, the
// rank and product of the pair each live position starts in registers (rk,
// md), the symbols in LDS at [position][lane] (lsym: this wave's L x 64
// words). Every byte has an id (the engine's all_bytes flag). A step costs
// a few instructions per position of L, so each class takes the smallest
// instance that holds it (4, 8, 12, 16; a 6 gained nothing, a 10 spilled).
template <int L>
__device__ void lane_bpe(const DevTables& t, const DevWork& w, uint32_t* lsym,
                         int64_t a, int n, int lane) {
  uint32_t rk[L], md[L];
  uint32_t live = n > 0 ? (1u << n) - 1 : 0u;  // n <= 16
  bool done = n == 0;
  if (!done && t.ignore_merges) {
    // whole-piece vocabulary hit first (pretok_kernel.cu:921-943 role)
    const int32_t hit = vocab_lookup(t, w.text + a, n);
    if (hit >= 0) {
      lsym[lane] = (uint32_t)hit;
      live = 1u;
      done = true;
    }
  }
  {
    uint32_t by[L];
#pragma unroll
    for (int i = 0; i < L; ++i) by[i] = i < n ? w.text[a + i] : 0u;
#pragma unroll
    for (int i = 0; i < L; ++i) {
      rk[i] = RANK_INF;
      md[i] = 0;
      if (!done && i < n) lsym[i * 64 + lane] = (uint32_t)t.byte_id[by[i]];
      if (!done && i + 1 < n) {
        const uint64_t v = t.bytepair[(by[i] << 8) | by[i + 1]];
        if (v != ~0ULL) {
          rk[i] = (uint32_t)(v >> 32);
          md[i] = (uint32_t)v;
        }
      }
    }
  }
  for (;;) {
    uint32_t best = RANK_INF, mid = 0;
    int bi = 0;
#pragma unroll
    for (int i = 0; i < L - 1; ++i)
      if (rk[i] < best) {
        best = rk[i];
        mid = md[i];
        bi = i;
      }
    if (best == RANK_INF) break;  // this lane's piece is finished
    // bi absorbs the next live position nb; p and nn: its live neighbours
    // after the merge
    const int nb = __builtin_ctz(live & ~((2u << bi) - 1u));
    const uint32_t after = live & ~((2u << nb) - 1u);
    const uint32_t before = live & ((1u << bi) - 1u);
    const int nn = after ? __builtin_ctz(after) : -1;
    const int p = before ? 31 - __builtin_clz(before) : -1;
    live &= ~(1u << nb);
    lsym[bi * 64 + lane] = mid;
    uint32_t rp = RANK_INF, mp = 0, rb = RANK_INF, mb = 0;
    if (p >= 0 && !pair_find(t, lsym[p * 64 + lane], mid, &rp, &mp)) rp = RANK_INF;
    if (nn >= 0 && !pair_find(t, mid, lsym[nn * 64 + lane], &rb, &mb)) rb = RANK_INF;
#pragma unroll
    for (int i = 0; i < L; ++i) {
      rk[i] = i == p ? rp : i == bi ? rb : i == nb ? RANK_INF : rk[i];
      md[i] = i == p ? mp : i == bi ? mb : md[i];
    }
  }
#pragma unroll
  for (int i = 0; i < L; ++i)
    if (i < n)
      w.tok[a + i] = ((live >> i) & 1) ? (lsym[i * 64 + lane] & SYM_ID) : INVALID_ID;
}

// One piece of up to 32 bytes per group of K = 32 / P lanes (lanes Kj ..
// Kj + K - 1 hold the same piece, at a, n bytes; n == 0: none): the lane r =
// lane % K of the group keeps positions g = rP + i (i < P), the pair
// starting at each as a key rank << 5 | g and its product in registers, the
// symbols in LDS at [i][lane]. Each step the group's lanes agree on the
// piece's lowest key -- lowest rank, leftmost on ties, the HF order -- and
// its product with log2(K) DPP exchanges inside the quad; the lane holding
// the pair merges it, and the lanes holding the two changed pairs look them
// up. Needs every byte to have an id and the compact pair table (ranks
// below 2^19, so the keys fit 32 bits).
constexpr int DPP_QUAD_SWAP1 = 0xB1;  // quad_perm [1, 0, 3, 2]
constexpr int DPP_QUAD_SWAP2 = 0x4E;  // quad_perm [2, 3, 0, 1]
template <int ctrl>
__device__ __forceinline__ uint32_t quad_dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, ctrl, 0xF, 0xF, false);
}

template <int P>
__device__ __forceinline__ void group_bpe(const DevTables& t, const DevWork& w,
                                          uint32_t* lsym, int64_t a, int n,
                                          int lane) {
  constexpr int K = 32 / P;
  static_assert(K == 2 || K == 4, "a group is two or four lanes of a quad");
  const int r = lane & (K - 1), g0 = P * r, lb = lane - r;
  uint32_t rk[P], md[P];
  uint32_t live = n >= 32 ? ~0u : (1u << n) - 1u;  // the piece's positions
  bool done = n == 0;
  if (t.ignore_merges) {
    // whole-piece vocabulary hit first (pretok_kernel.cu:921-943 role), by
    // the group's first lane
    int32_t hit = -1;
    if (!done && r == 0) hit = vocab_lookup(t, w.text + a, n);
    hit = (int32_t)quad_dpp<K == 2 ? 0xA0 : 0x00>((uint32_t)hit);  // [0,0,2,2] / [0,0,0,0]
    if (!done && hit >= 0) {
      if (r == 0) lsym[lane] = (uint32_t)hit;
      live = 1u;
      done = true;
    }
  }
  {
    uint32_t by[P + 1];
#pragma unroll
    for (int i = 0; i < P + 1; ++i) {
      by[i] = g0 + i < n ? w.text[a + g0 + i] : 0u;
    }
#pragma unroll
    for (int i = 0; i < P; ++i) {
      rk[i] = RANK_INF;
      md[i] = 0;
      if (!done && g0 + i < n) lsym[i * 64 + lane] = (uint32_t)t.byte_id[by[i]];
      if (!done && g0 + i + 1 < n) {
        const uint64_t v = t.bytepair[(by[i] << 8) | by[i + 1]];
        if (v != ~0ULL) {
          rk[i] = (uint32_t)(v >> 32) << 5 | (uint32_t)(g0 + i);
          md[i] = (uint32_t)v;
        }
      }
    }
  }
  for (;;) {
    // this lane's lowest key and its product, then the group's (keys are
    // distinct: each holds its position)
    uint32_t km = RANK_INF, mid = 0;
#pragma unroll
    for (int i = 0; i < P; ++i) {
      if (rk[i] < km) {
        km = rk[i];
        mid = md[i];
      }
    }
    {
      const uint32_t ko = quad_dpp<DPP_QUAD_SWAP1>(km), mo = quad_dpp<DPP_QUAD_SWAP1>(mid);
      if (ko < km) { km = ko; mid = mo; }
    }
    if constexpr (K == 4) {
      const uint32_t ko = quad_dpp<DPP_QUAD_SWAP2>(km), mo = quad_dpp<DPP_QUAD_SWAP2>(mid);
      if (ko < km) { km = ko; mid = mo; }
    }
    if (km == RANK_INF) break;  // this group's piece is finished
    const int bi = (int)(km & 31);
    const bool own_b = bi / P == r;
    // bi absorbs the next live position nb (bi <= 30); p and nn: its live
    // neighbours after the merge
    const int nb = __builtin_ctz(live & ~((2u << bi) - 1u));
    const uint32_t after = live & ~((2u << nb) - 1u);  // (nb == 31: none)
    const uint32_t before = live & ((1u << bi) - 1u);
    const int nn = after ? __builtin_ctz(after) : -1;
    const int p = before ? 31 - __builtin_clz(before) : -1;
    live &= ~(1u << nb);
    if (own_b) lsym[(bi % P) * 64 + lane] = mid;
    uint32_t rp = RANK_INF, mp = 0, rb = RANK_INF, mb = 0, r_, m_;
    if (p >= 0 && p / P == r &&
        ctab_find(t, lsym[(p % P) * 64 + lane], mid, &r_, &m_)) {
      rp = r_ << 5 | (uint32_t)p;
      mp = m_;
    }
    if (nn >= 0 && own_b &&
        ctab_find(t, mid, lsym[(nn % P) * 64 + lb + nn / P], &r_, &m_)) {
      rb = r_ << 5 | (uint32_t)bi;
      mb = m_;
    }
    // (positions relative to this lane's first)
    const int pl = p - g0, bl = bi - g0, nl = nb - g0;
#pragma unroll
    for (int i = 0; i < P; ++i) {
      rk[i] = i == pl ? rp : i == bl ? rb : i == nl ? RANK_INF : rk[i];
      md[i] = i == pl ? mp : i == bl ? mb : md[i];
    }
  }
#pragma unroll
  for (int i = 0; i < P; ++i) {
    if (g0 + i < n)
      w.tok[a + g0 + i] =
          ((live >> (g0 + i)) & 1) ? (lsym[i * 64 + lane] & SYM_ID) : INVALID_ID;
  }
}

// geometry word of a class: slot | pieces per unit << 8 | pack_magic << 16 |
// lanes per piece << 28
constexpr uint32_t pack_geo(int c) {
  return (uint32_t)pack_slot(c) | (uint32_t)pack_per_unit(c) << 8 |
         (uint32_t)pack_magic(c) << 16 | (uint32_t)pack_lanes(c) << 28;
}
__constant__ uint32_t PACK_GEO[PACK_CLASSES] = {
    pack_geo(0), pack_geo(1), pack_geo(2), pack_geo(3), pack_geo(4),
    pack_geo(5), pack_geo(6), pack_geo(7), pack_geo(8), pack_geo(9),
    pack_geo(10), pack_geo(11), pack_geo(12)};
static_assert(PACK_CLASSES == 13, "PACK_GEO lists every class");

// Long pieces (k_pretok queued their starts), entries k0..k0+63 of the
// queue by one wave: their ends, and the pieces over WIDE_MAX bytes -- a
// whole-vocabulary hit (ignore_merges), else (certification on) their
// bytes marked in inlong for the cut / segment / certify stages. Returns
// how many are over WIDE_MAX bytes, and adds to nrows and nwide how many
// have 129..256 and 257..WIDE_MAX (wave-uniform).
constexpr int WIDE_MAX = 512;
__device__ __forceinline__ uint32_t long_prep_step(const DevTables& t,
                                                   const DevWork& w,
                                                   uint32_t k0, uint32_t n,
                                                   int lane, uint32_t& nrows,
                                                   uint32_t& nwide) {
  const uint32_t k = k0 + lane;
  uint32_t a = 0, b = 0;
  bool far = false;
  if (k < n) {
    // the end is the next start bit, found here when it lies in the
    // piece's first two words
    a = w.longlist[2 * k];
    const int64_t wd = a >> 6;
    const uint64_t gt = w.starts[wd] & ~mask_le((int)(a & 63));
    const uint64_t nx = w.starts[wd + 1];
    if (gt) b = (uint32_t)(wd * 64 + __builtin_ctzll(gt));
    else if (nx) b = (uint32_t)((wd + 1) * 64 + __builtin_ctzll(nx));
    else far = true;
  }
  // longer pieces (the words pretok wrote end at nwords, and the word
  // holding byte nb has a start bit at or after nb, so every search ends
  // before them). Eight at a time first: lane group g (lanes 8g..8g+7)
  // reads words 2..9 of the g-th pending piece, one load a lane, which
  // ends every piece of up to ~576 bytes (one dependent load for eight
  // pieces instead of one each: a wave of C5's 129-256-byte pieces has
  // fifty of them, and the gate opens after its slowest wave).
  const int64_t nwords = (w.nb + 63) / 64 + 2;
  uint64_t rest = 0;
  for (uint64_t pend = __ballot(far); pend;) {
    const int g = lane >> 3, sub = lane & 7;
    uint64_t p = pend;
    for (int q = 0; q < g && p; ++q) p &= p - 1;
    const int j = p ? __builtin_ctzll(p) : 0;
    const uint32_t pa = __shfl(a, j);
    const int64_t wq = (int64_t)(pa >> 6) + 2 + sub;
    const uint64_t word = !p ? 0ULL : wq < nwords ? w.starts[wq] : ~0ULL;
    const uint32_t gm = (uint32_t)(__ballot(word != 0) >> (8 * g)) & 0xFFu;
    const int l = gm ? __builtin_ctz(gm) : 0;
    const uint64_t wl = __shfl(word, 8 * g + l);
    const uint32_t ge = (uint32_t)(((pa >> 6) + 2 + l) * 64 + __builtin_ctzll(wl | (1ULL << 63)));
    // each pending lane among the first eight takes its group's result
    const uint32_t r = (uint32_t)__popcll(pend & ((1ULL << lane) - 1));
    const bool mine = ((pend >> lane) & 1) && r < 8;
    const uint32_t e8 = (uint32_t)__shfl((int)ge, 8 * (int)(r & 7));
    const bool ok8 = __shfl((int)gm, 8 * (int)(r & 7)) != 0;
    if (mine && ok8) b = e8;
    rest |= __ballot(mine && !ok8);
    for (int q = 0; q < 8 && pend; ++q) pend &= pend - 1;
  }
  // the rest, one after another: the wave reads 64 words at a time
  for (uint64_t pend = rest; pend; pend &= pend - 1) {
    const int j = __builtin_ctzll(pend);
    const uint32_t pa = __shfl(a, j);
    uint32_t end = 0;
    for (int64_t wd = (pa >> 6) + 10;; wd += 64) {
      const uint64_t word = wd + lane < nwords ? w.starts[wd + lane] : ~0ULL;
      const uint64_t nz = __ballot(word != 0);
      if (nz) {
        const int l = __builtin_ctzll(nz);
        const uint64_t wl = __shfl(word, l);
        end = (uint32_t)((wd + l) * 64 + __builtin_ctzll(wl));
        break;
      }
    }
    if (lane == j) b = end;
  }
  if (k < n) w.longlist[2 * k + 1] = b;
  nrows += (uint32_t)__popcll(__ballot(k < n && b - a > 128u && b - a <= 256u));
  nwide += (uint32_t)__popcll(
      __ballot(k < n && b - a > 256u && b - a <= (uint32_t)WIDE_MAX));
  uint64_t big = __ballot(k < n && b - a > (uint32_t)WIDE_MAX);
  const uint32_t nbig = (uint32_t)__popcll(big);
  while (big) {  // wave-uniform
    const int j = __builtin_ctzll(big);
    big &= big - 1;
    const uint32_t pa = __shfl(a, j), pb = __shfl(b, j);
    if (t.ignore_merges) {
      int32_t hit = -1;
      if (lane == 0) hit = vocab_lookup(t, w.text + pa, (int64_t)(pb - pa));
      hit = __shfl(hit, 0);
      if (hit >= 0) {
        for (uint32_t p = pa + lane; p < pb; p += 64)
          w.tok[p] = p == pa ? (uint32_t)hit : INVALID_ID;
        continue;
      }
    }
    if (!t.cert) continue;  // merged whole by k_seg_block (mode 1)
    // mark the piece's bytes: whole words directly, the two edge words
    // (shared with neighbouring pieces) with an atomic OR
    const uint32_t wa = pa >> 6, wb = (pb - 1) >> 6;
    for (uint32_t wd = wa + lane; wd <= wb; wd += 64) {
      const uint32_t lo = wd == wa ? (pa & 63) : 0;
      const uint32_t hi = wd == wb ? ((pb - 1) & 63) + 1 : 64;
      const uint64_t m = lanes_in((int)lo, (int)hi);
      if (m == ~0ULL) w.inlong[wd] = m;
      else atomicOr(reinterpret_cast<unsigned long long*>(&w.inlong[wd]), m);
    }
  }
  return nbig;
}

// (defined with the long-piece merges below)
template <int R, bool H = false>
__device__ __forceinline__ void wave_bpe_rows(const DevTables& t,
                                              const DevWork& w, uint32_t a,
                                              int len, bool vocab_first,
                                              const uint32_t* unsafe_lds,
                                              const uint4* hot = nullptr);

// Work units by class: pack_per_unit(c) pieces of class c each. Workgroups
// go to the XCDs in turn (block b on XCD b % PACK_XCDS, up to a rotation),
// as k_pretok's did, and each XCD has its own L2: so the blocks of residue x
// merge segment x of the lists, the pieces of the tiles that XCD
// pretokenized (whose text and start words it last read). An XCD's units go
// in one order, class by class, longest merge chains first (PACK_ORDER, from
// the per-class unit times of a cycle-counter probe build: the 17..32-byte
// groups and the 9..16-byte lanes first). Wave g of the XCD's G waves takes
// unit g first; every later unit comes from the segment's counter (G plus
// the count so far, which starts at 0 in each call's control slot), one at
// a time as waves finish theirs. Ahead of the classes in every XCD's order
// come the queued long pieces of 65..128 bytes (entries k of the long-piece
// queue with k % PACK_XCDS == x), one per unit, merged by the wave with its
// state in registers (wave_bpe_rows): the longest chains of all. (Longer
// ones go to the side streams: the 256-byte instance does not fit this
// kernel's registers; so do these when more than PACK_ROWS_MAX pieces are
// queued, where they would lengthen this kernel more than the side
// stream's join costs.)
// The long units thus all start at once, and the SIMDs end on the short
// ones, each SIMD busy until its share is done (with a fixed share per wave
// a SIMD holding a few long units ran on alone, latency-bound, long after
// the others). Classes of up to PACK_LANE_MAX bytes: 64 pieces per unit,
// one per lane (lane_bpe); up to 32 bytes: 16 pieces per unit, four lanes
// each (group_bpe); longer ones, and every class of a table without an id
// for every byte or without the compact pair table: 64 / slot pieces at a
// time, a slot of lanes each (wave_bpe). (Groups of eight lanes for 33..64
// bytes were slower: one merge per step makes their units the longest
// chains of the launch, where one piece per wave merges every occurrence of
// a rank per round.)
__constant__ int8_t PACK_ORDER[PACK_CLASSES] = {11, 9, 10, 8, 7, 6, 5, 12,
                                                4, 3, 2, 1, 0};
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8, 8)))
void k_bpe_pack(DevTables t, DevWork w) {
  __shared__ uint32_t lds[4][PACK_LANE_MAX * 64];
  // the unit order of this block's segment, built by wave 0: mo[k] = the
  // first unit of the k-th class of the order, mk[k] = the class
  // (PACK_CLASSES: the long pieces, k = 0); mg2[c] = class c's piece count
  // and geometry (slot | pieces per unit << 8 | pack_magic << 16 | lane /
  // group flags), ml[c] = the start of its list; mtot = the segment's
  // units. Kept in LDS, not registers: the merge paths need every register
  // they can get.
  __shared__ uint32_t mo[16];
  __shared__ uint2 mg2[16];
  __shared__ uint32_t ml[16];
  __shared__ int32_t mk[16];
  __shared__ uint32_t mtot;
  const int lane = threadIdx.x & 63, wv = wave_id();
  const bool cl = lane < PACK_CLASSES;
  const int x = blockIdx.x % PACK_XCDS;
  const uint32_t* const seg = w.pseg + x * CTRL_PSEG_STRIDE;
  uint32_t nl = *w.longcount;  // queued long pieces
  if (nl > w.long_cap) nl = w.long_cap;
  if (wv == 0) {
    const uint32_t cnt = cl ? seg[CTRL_PSEG_COUNT + lane] : 0u;
    const uint32_t geo = cl ? PACK_GEO[lane] : 0u;
    const uint32_t per = cl ? (geo >> 8) & 0xFF : 1u;
    const uint32_t nu = (cnt + per - 1) / per;  // the class's units
    // order position k: 0 the long pieces, k >= 1 class PACK_ORDER[k - 1]
    const bool ko = lane <= PACK_CLASSES;
    const int oc = lane == 0 ? PACK_CLASSES : ko ? PACK_ORDER[lane - 1] : 0;
    const uint32_t nuo = (uint32_t)__shfl((int)nu, oc);
    const uint32_t nr = nl <= (uint32_t)PACK_ROWS_MAX && nl > (uint32_t)x
                            ? (nl - x + PACK_XCDS - 1) / PACK_XCDS : 0u;
    const uint32_t lk = lane == 0 ? nr : ko ? nuo : 0u;
    const uint32_t incl = wave_incl_scan(lk, lane);
    if (lane < 16) {
      mo[lane] = ko ? incl - lk : ~0u;
      mk[lane] = oc;
      mg2[lane] = make_uint2(cnt, geo);
      ml[lane] = cl ? pack_seg_list((uint32_t)pretok_tiles(w.nb), x,
                                    PACK_LOCAL_OFF[lane])
                    : 0u;
    }
    const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    if (lane == 0) mtot = tot;
  }
  __syncthreads();
  {
    // The long pieces first, 64 a wave, by the first waves of the grid
    // (long_prep_step). The last of them opens the gate: how many pieces
    // are over 64 bytes and how many over WIDE_MAX, then the call's number
    // (with no long piece, wave 0 of block 0 does).
    constexpr uint32_t GW = PACK_BLOCKS * 4;
    const uint32_t n = nl;
    const uint32_t P = (n + 63) / 64 < GW ? (n + 63) / 64 : GW;
    const uint32_t gw = blockIdx.x * 4 + wv;
    if (gw < P || (P == 0 && gw == 0)) {
      uint32_t big = 0, rows = 0, wide = 0;
      for (uint32_t k0 = gw * 64; k0 < n; k0 += GW * 64)
        big += long_prep_step(t, w, k0, n, lane, rows, wide);
      if (lane == 0) {
        bool last = true;
        if (P) {
          if (big) atomicAdd(w.nbig, big);
          if (rows) atomicAdd(w.nrows, rows);
          if (wide) atomicAdd(w.nwide, wide);
          __threadfence();
          last = atomicAdd(w.prepdone, 1u) == P - 1;
        }
        if (last && w.gate) {
          __threadfence();
          w.gate[GATE_NLONG] = n;
          w.gate[GATE_NROWS] = __hip_atomic_load(w.nrows, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
          w.gate[GATE_NWIDE] = __hip_atomic_load(w.nwide, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
          w.gate[GATE_BIG] = __hip_atomic_load(w.nbig, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
          __threadfence_system();
          w.gate[GATE_SEQ] = w.seq;
          __threadfence_system();
        }
      }
    }
  }
  // (values read from LDS are wave-uniform here: readfirstlane keeps them
  // in scalar registers)
  const uint32_t total = __builtin_amdgcn_readfirstlane(mtot);
  uint32_t* const queue = w.pseg + x * CTRL_PSEG_STRIDE;
  constexpr uint32_t G = (PACK_BLOCKS / PACK_XCDS) * 4;  // waves per XCD
  uint32_t u0 = (blockIdx.x / PACK_XCDS) * 4 + wv;  // the first unit
  for (bool first_unit = true;; first_unit = false) {
    if (!first_unit) {
      // the next unit of the segment's order (a vector atomic by lane 0)
      uint32_t got = 0;
      if (lane == 0)
        got = __hip_atomic_fetch_add(queue, 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
      u0 = G + __builtin_amdgcn_readfirstlane(got);
    }
    if (u0 >= total) break;  // every wave leaves once the units are taken
    // The lane index, opaque to the compiler for each unit: without it the
    // per-lane LDS addresses of the merge paths are hoisted out of this
    // loop, and holding them across it spills registers to scratch (a few
    // MB of scratch written back per launch).
    int lane_u = lane;
    asm volatile("" : "+v"(lane_u));
    // the unit's place in the order: the last class whose first unit is at
    // or before u0 (a class without units shares the next one's first unit)
    const uint32_t m = lane_u <= PACK_CLASSES ? mo[lane_u] : ~0u;
    const uint64_t le = __ballot(m <= u0);
    const int ko = 63 - __builtin_clzll(le);
    const uint32_t kbeg = __builtin_amdgcn_readlane(m, ko);
    const int c = __builtin_amdgcn_readfirstlane(mk[ko]);
    if (c == PACK_CLASSES) {  // wave-uniform: a queued long piece
      // its end is the next start bit, looked for here in the next 128
      // bytes (the first waves may not have written it yet); a piece
      // without one there is longer, left to the side streams, and a
      // sentinel bit ends the search at the text's end
      const uint32_t a = w.longlist[2 * ((u0 - kbeg) * PACK_XCDS + x)];
      int len = 129;
      {
        const int64_t wd = a >> 6;
        uint64_t word = w.starts[wd] & ~mask_le((int)(a & 63));
#pragma unroll
        for (int j = 1; j <= 3 && len > 128; ++j) {
          if (word) {
            const int64_t e = (wd + j - 1) * 64 + __builtin_ctzll(word);
            len = e - a <= 128 ? (int)(e - a) : 129;
            break;
          }
          word = w.starts[wd + j];
        }
      }
      if (len > 64 && len <= 128) wave_bpe_rows<2>(t, w, a, len, true, nullptr);
      continue;
    }
    const uint2 gc = mg2[c];
    const uint32_t cnt = __builtin_amdgcn_readfirstlane(gc.x);
    const uint32_t geo = __builtin_amdgcn_readfirstlane(gc.y);
    const uint32_t* const list = w.plist + __builtin_amdgcn_readfirstlane(ml[c]);
    const int sl = geo & 0xFF, k = (geo >> 8) & 0xFF, mg = (geo >> 16) & 0xFFF;
    const uint32_t first = (u0 - kbeg) * k;  // the unit's first piece
    const int lanes = (int)(geo >> 28);
    if (lanes == 1 && t.all_bytes) {  // wave-uniform
      const uint32_t idx = first + lane_u;
      int64_t a = 0;
      int n = 0;
      if (idx < cnt) {
        a = list[idx];
        n = (int)(piece_end(w, a) - a);
      }
      uint32_t* ls = lds[wv];
      if (sl <= 4) lane_bpe<4>(t, w, ls, a, n, lane_u);
      else if (sl <= 8) lane_bpe<8>(t, w, ls, a, n, lane_u);
      else if (sl <= 12) lane_bpe<12>(t, w, ls, a, n, lane_u);
      else lane_bpe<16>(t, w, ls, a, n, lane_u);
      continue;
    }
    if (lanes == 4 && t.all_bytes && t.ctab) {  // wave-uniform
      const uint32_t idx = first + (uint32_t)(lane_u / lanes);
      int64_t a = 0;
      int n = 0;
      if (idx < cnt) {
        a = list[idx];
        n = (int)(piece_end(w, a) - a);
      }
      group_bpe<8>(t, w, lds[wv], a, n, lane_u);
      continue;
    }
    // slot-packed: 64 / slot pieces at a time (a lane-class unit without
    // the lane path takes several passes)
    const int per = 64 / sl;
    const int slot = (lane_u * mg) >> 12, off = lane_u - slot * sl;
    for (int j0 = 0; j0 < k; j0 += per) {
      const uint32_t idx = first + j0 + slot;
      int64_t a = 0, L = 0;
      if (slot < per && j0 + slot < k && idx < cnt) {
        a = list[idx];
        L = piece_end(w, a) - a;
      }
      const bool elig = off < L;
      const int ps = elig ? slot * sl : lane_u, pe = elig ? slot * sl + (int)L : lane_u + 1;
      wave_bpe<true, false, true>(t, w, 0, a + off, lane_u, elig, ps, pe);
    }
  }
}

hipError_t launch_bpe_pack(const DevTables& t, const DevWork& w, hipStream_t s,
                           hipEvent_t start, hipEvent_t stop) {
  launch_ev(k_bpe_pack, dim3(PACK_BLOCKS), dim3(256), s, start, stop, t, w);
  return hipGetLastError();
}

// ------------------------------------------------- 3. long-piece BPE
//
// A piece longer than 64 bytes is cut into short segments at positions that
// are token boundaries in the BPE of a 64-byte window centred on them; the
// segments are merged independently (wave per window, recording how each
// segment's first and last token evolve); then every cut is certified:
// with a merge table in which every rule that consumes a token ranks above
// every rule that makes it, the whole-piece process is the rank-ordered
// interleaving of the segment processes as long as no pair across a cut is
// ever merged, and whether it is can be decided from the two boundary
// histories alone (the pair across the cut at each moment, against the
// ranks at which its two tokens are next consumed). A failed cut is
// removed and the joined segment redone, until every remaining cut holds;
// the worst case is the whole piece as one segment. Tables with a rule
// out of that order are certified from every merge round; with bytes
// without an id, pieces are merged whole. Segments (and such pieces) over
// WIDE_MAX bytes are merged by a workgroup each (block_bpe).


// ---- wide pieces: one wave per piece / segment of 65..WIDE_MAX bytes,
// state in LDS (slot s = 64*row + lane). Each round merges every leftmost
// non-overlapping occurrence of the lowest-ranked pair at once, which is the
// one-at-a-time order when that rank's result is consumed only by higher
// ranks; a rank flagged in unsafe_bits merges its leftmost occurrence
// alone (src/toktier/kernels/bpe_tables.py:435-501 guard,
// pretok_kernel.cu:1174-1186).
constexpr int WIDE_ROWS = WIDE_MAX / 64;
constexpr uint32_t SYM_RAW = 0x80000000u;  // symbol is still its raw byte

struct WideLds {
  uint32_t sym[WIDE_MAX];
  uint32_t rk[WIDE_MAX];
  uint32_t mid[WIDE_MAX];
  int16_t nx[WIDE_MAX];
  int16_t pv[WIDE_MAX];
};

__device__ __forceinline__ void lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
}

__device__ __forceinline__ bool rank_unsafe(const DevTables& t, uint32_t r) {
  return t.unsafe && ((r >> 5) < t.unsafe_words) &&
         ((t.unsafe[r >> 5] >> (r & 31)) & 1);
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) v = min(v, (uint32_t)__shfl_xor(v, d));
  return v;
}

// ---- segments over WIDE_MAX bytes: one workgroup each
//
// block_bpe merges the segment [a, b) in the HF order with the guarded
// batch rounds of wave_bpe_wide: each round takes the lowest-ranked pair; a
// safe rank merges every leftmost non-overlapping occurrence at once, an
// unsafe one its leftmost alone. Its state lives in the segment's per-byte
// scratch: tok (the symbol at its first byte, INVALID_ID elsewhere), nx /
// pv (the neighbouring symbols), and in heap (3 words per byte) each
// symbol's pair (rank << 32 | product id), the round that selected it, and
// per 1024-byte chunk the lowest key (rank << 32 | offset; SEGB_NOPAIR
// ranks a symbol with no pair, all ones a chunk with no symbol) and the
// round that last touched it. A round reads the chunk minima, scans only
// the chunks that hold its rank (taking a pair when the pair before it was
// not taken: a two-state automaton composed over the block), merges, and
// recomputes the pairs and minima of the chunks it touched. Histories as
// wave_bpe_wide's (a record per round for certification from every round,
// else the first / last-token events).
constexpr int SEGB_TPB = 1024;
constexpr int SEGB_WAVES = SEGB_TPB / 64;
constexpr uint32_t SEGB_NOPAIR = 0xFFFFFFFEu;
// the selection automaton's functions of the previous pair's "taken" bit:
// bit x is the image of x
constexpr uint32_t SF_ID = 2, SF_ZERO = 0, SF_NOT = 1;
__device__ __forceinline__ uint32_t sf_at(uint32_t f, uint32_t x) { return (f >> x) & 1; }
__device__ __forceinline__ uint32_t sf_then(uint32_t f, uint32_t g) {
  return sf_at(g, sf_at(f, 0)) | (sf_at(g, sf_at(f, 1)) << 1);
}
struct SegLds {
  uint64_t wmin[SEGB_WAVES];
  uint32_t wfn[SEGB_WAVES];
  uint32_t queue[SEGB_TPB];
  uint32_t nq;
  int32_t hit, last;
};

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor((uint32_t)v, m), hi = __shfl_xor((uint32_t)(v >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}

// the workgroup's lowest 64-bit key, in every thread
__device__ uint64_t block_min64(uint64_t v, SegLds& L) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const uint64_t o = shfl_xor64(v, d);
    v = o < v ? o : v;
  }
  if (lane == 0) L.wmin[wv] = v;
  __syncthreads();
  uint64_t m = L.wmin[0];
  for (int i = 1; i < SEGB_WAVES; ++i) m = L.wmin[i] < m ? L.wmin[i] : m;
  __syncthreads();
  return m;
}

// a symbol's key in its chunk's minimum
__device__ __forceinline__ uint64_t segb_key(uint64_t pair, uint32_t off) {
  const uint32_t r = pair == ~0ULL ? SEGB_NOPAIR : (uint32_t)(pair >> 32);
  return ((uint64_t)r << 32) | off;
}

__device__ void block_bpe(const DevTables& t, const DevWork& w, uint32_t a,
                          uint32_t b, bool vocab_first, bool hist, SegLds& L) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t n = b - a;
  const uint32_t nch = (n + SEGB_TPB - 1) / SEGB_TPB;
  uint64_t* pair = w.heap + 3ull * a;
  uint32_t* selr = reinterpret_cast<uint32_t*>(pair + n);
  uint32_t* dirty = selr + n;
  uint64_t* cmin = pair + 2ull * n;
  uint32_t* tok = w.tok;
  int32_t* nx = w.nx;
  int32_t* pv = w.pv;
  if (vocab_first && t.ignore_merges) {
    if (tid == 0) L.hit = vocab_lookup(t, w.text + a, (int64_t)n);
    __syncthreads();
    const int32_t hit = L.hit;
    __syncthreads();
    if (hit >= 0) {
      for (uint32_t i = tid; i < n; i += SEGB_TPB)
        tok[a + i] = i == 0 ? (uint32_t)hit : INVALID_ID;
      return;
    }
  }
  for (uint32_t i = tid; i < n; i += SEGB_TPB) {
    const int32_t id = t.byte_id[w.text[a + i]];
    tok[a + i] = id >= 0 ? (uint32_t)id : INVALID_ID;
    selr[i] = 0;
  }
  for (uint32_t c = tid; c < nch; c += SEGB_TPB) dirty[c] = 0;
  __syncthreads();
  // neighbour links over the symbols (bytes without an id dropped)
  for (uint32_t i = tid; i < n; i += SEGB_TPB) {
    if (tok[a + i] == INVALID_ID) continue;
    uint32_t j = i + 1;
    while (j < n && tok[a + j] == INVALID_ID) ++j;
    nx[a + i] = j < n ? (int32_t)(a + j) : -1;
    int64_t q = (int64_t)i - 1;
    while (q >= 0 && tok[a + q] == INVALID_ID) --q;
    pv[a + i] = q >= 0 ? (int32_t)(a + q) : -1;
  }
  __syncthreads();
  // pairs and chunk minima; the first and the last symbol
  uint64_t fst = ~0ULL, lst = ~0ULL;
  for (uint32_t c = 0; c < nch; ++c) {
    const uint32_t i = c * SEGB_TPB + tid;
    uint64_t k = ~0ULL;
    if (i < n && tok[a + i] != INVALID_ID) {
      const int32_t q = nx[a + i];
      const uint64_t v = q >= 0 ? pair_lookup(t, tok[a + i], tok[q]) : ~0ULL;
      pair[i] = v;
      k = segb_key(v, i);
      fst = fst < i ? fst : i;
      lst = lst < (uint64_t)(n - 1 - i) ? lst : (uint64_t)(n - 1 - i);
    }
    const uint64_t m = block_min64(k, L);
    if (tid == 0) cmin[c] = m;
  }
  fst = block_min64(fst, L);
  lst = block_min64(lst, L);
  if (fst == ~0ULL) {  // no symbol at all
    if (hist && tid == 0) w.hmeta[a] = 0;
    return;
  }
  const uint32_t first = (uint32_t)fst;
  if (tid == 0) L.last = (int32_t)(n - 1 - (uint32_t)lst);
  uint32_t nfirst = 0, nlast = 0;  // (thread 0's)
  for (uint32_t round = 1;; ++round) {
    uint64_t m = ~0ULL;
    for (uint32_t c = tid; c < nch; c += SEGB_TPB) m = cmin[c] < m ? cmin[c] : m;
    m = block_min64(m, L);
    const uint32_t R = (uint32_t)(m >> 32);
    if (R >= SEGB_NOPAIR) break;
    // every round merges at least its leftmost lowest pair, so n rounds
    // end it; past that the state is broken: report it, never spin
    if (round > n) {
      if (tid == 0) atomicOr(w.status, ST_ROUNDS);
      break;
    }
    const uint32_t s0 = (uint32_t)m;
    const uint32_t prod = (uint32_t)pair[s0];
    const bool single = rank_unsafe(t, R);
    // the selection
    if (single) {
      if (tid == 0) selr[s0] = round;
    } else {
      uint32_t carry = 0;  // the pair before the chunk was taken
      for (uint32_t c = 0; c < nch; ++c) {
        const uint64_t cm = cmin[c];
        if ((uint32_t)(cm >> 32) != R) {
          if (cm != ~0ULL) carry = 0;  // its last symbol's pair is not taken
          continue;
        }
        const uint32_t i = c * SEGB_TPB + tid;
        uint32_t fn = SF_ID;
        if (i < n && tok[a + i] != INVALID_ID)
          fn = (pair[i] != ~0ULL && (uint32_t)(pair[i] >> 32) == R) ? SF_NOT : SF_ZERO;
        uint32_t F = fn;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          const uint32_t o = __shfl_up(F, d);
          if (lane >= d) F = sf_then(o, F);
        }
        if (lane == 63) L.wfn[wv] = F;
        __syncthreads();
        uint32_t P = SF_ID, T = SF_ID;
        for (int j = 0; j < SEGB_WAVES; ++j) {
          if (j < wv) P = sf_then(P, L.wfn[j]);
          T = sf_then(T, L.wfn[j]);
        }
        __syncthreads();
        uint32_t E = __shfl_up(F, 1);
        if (lane == 0) E = SF_ID;
        const uint32_t in = sf_at(sf_then(P, E), carry);
        if (fn == SF_NOT && !in) selr[i] = round;
        carry = sf_at(T, carry);
      }
    }
    __syncthreads();
    if (hist && tid == 0) {
      const int32_t l = L.last;
      const int32_t pl = pv[a + l] >= 0 ? pv[a + l] - (int32_t)a : -1;
      const bool fsel = selr[first] == round;
      const bool lsel = pl >= 0 && selr[pl] == round;
      if (t.cert == 2) {
        w.hfirst[a + nfirst++] = ((uint64_t)R << 32) | (fsel ? HR_FIRST : 0) |
                                 (lsel ? HR_LAST : 0) | prod;
      } else {
        if (fsel) w.hfirst[a + nfirst++] = ((uint64_t)R << 32) | prod;
        if (lsel) w.hlast[a + nlast++] = ((uint64_t)R << 32) | prod;
      }
      if (lsel) L.last = pl;
    }
    // the merges: a selected symbol takes its right neighbour (a symbol
    // without one, or one already merged away, means a broken state:
    // reported, and nothing is written through its stale links)
    auto merge = [&](uint32_t i) {
      const int32_t p = (int32_t)(a + i), q = nx[p];
      if (q < (int32_t)a || q >= (int32_t)b || tok[p] == INVALID_ID ||
          tok[q] == INVALID_ID) {
        atomicOr(w.status, ST_ROUNDS);
        return;
      }
      const int32_t nn = nx[q];
      tok[p] = prod;
      tok[q] = INVALID_ID;
      nx[p] = nn;
      if (nn >= 0) pv[nn] = p;
      dirty[i / SEGB_TPB] = round;
      dirty[(uint32_t)(q - (int32_t)a) / SEGB_TPB] = round;
      const int32_t pp = pv[p];
      if (pp >= 0) dirty[(uint32_t)(pp - (int32_t)a) / SEGB_TPB] = round;
    };
    if (single) {
      if (tid == 0) merge(s0);
    } else {
      for (uint32_t c = 0; c < nch; ++c) {
        if ((uint32_t)(cmin[c] >> 32) != R) continue;
        const uint32_t i = c * SEGB_TPB + tid;
        if (i < n && selr[i] == round) merge(i);
      }
    }
    __syncthreads();
    // the pairs that changed (the selected symbols and the symbols before
    // them) and the minima of the chunks touched
    for (uint32_t c = 0; c < nch; ++c) {
      if (dirty[c] != round) continue;
      const uint32_t i = c * SEGB_TPB + tid;
      uint64_t k = ~0ULL;
      if (i < n && tok[a + i] != INVALID_ID) {
        const int32_t q = nx[a + i];
        if (selr[i] == round || (q >= 0 && selr[q - (int32_t)a] == round))
          pair[i] = q >= 0 ? pair_lookup(t, tok[a + i], tok[q]) : ~0ULL;
        k = segb_key(pair[i], i);
      }
      const uint64_t mc = block_min64(k, L);
      if (tid == 0) cmin[c] = mc;
    }
    // thread 0's last chunk minimum must be written before the next round
    // reads the minima (thread c reads chunk c's before any barrier)
    __syncthreads();
  }
  if (hist && tid == 0) w.hmeta[a] = t.cert == 2 ? nfirst : nfirst | (nlast << 16);
  __syncthreads();
}

// pair value for the symbols at slots s and n of a piece starting at a
__device__ __forceinline__ uint64_t wide_pair(const DevTables& t,
                                              const DevWork& w, uint32_t a,
                                              const WideLds& L, int s, int n) {
  const uint32_t x = L.sym[s], y = L.sym[n];
  if ((x & y) & SYM_RAW)
    return t.bytepair[((uint32_t)w.text[a + s] << 8) | w.text[a + n]];
  return pair_lookup(t, x & ~SYM_RAW, y & ~SYM_RAW);
}

__device__ void wave_bpe_wide(const DevTables& t, const DevWork& w,
                              uint32_t a, int len, bool vocab_first,
                              bool hist, WideLds& L) {
  const int lane = threadIdx.x & 63;
  const int rows = (len + 63) >> 6;
  if (vocab_first && t.ignore_merges) {
    int32_t hit = -1;
    if (lane == 0) hit = vocab_lookup(t, w.text + a, len);
    hit = __shfl(hit, 0);
    if (hit >= 0) {
      for (int r = 0; r < rows; ++r) {
        const int s = r * 64 + lane;
        if (s < len) w.tok[a + s] = s == 0 ? (uint32_t)hit : INVALID_ID;
      }
      return;
    }
  }
  uint64_t live[WIDE_ROWS];
#pragma unroll
  for (int r = 0; r < WIDE_ROWS; ++r) {
    const int s = r * 64 + lane;
    int32_t id = -1;
    if (r < rows && s < len) id = t.byte_id[w.text[a + s]];
    if (r < rows) L.sym[s] = id >= 0 ? (SYM_RAW | (uint32_t)id) : 0u;
    live[r] = __ballot(id >= 0);
  }
  // neighbour links over the live slots
#pragma unroll
  for (int r = 0; r < WIDE_ROWS; ++r) {
    if (r >= rows) break;
    const int s = r * 64 + lane;
    int n = -1, p = -1;
    uint64_t m = live[r] & ~mask_le(lane);
    if (m) n = r * 64 + __builtin_ctzll(m);
    for (int q = r + 1; n < 0 && q < rows; ++q)
      if (live[q]) n = q * 64 + __builtin_ctzll(live[q]);
    m = live[r] & ((1ULL << lane) - 1);
    if (m) p = r * 64 + 63 - __builtin_clzll(m);
    for (int q = r - 1; p < 0 && q >= 0; --q)
      if (live[q]) p = q * 64 + 63 - __builtin_clzll(live[q]);
    L.nx[s] = (int16_t)n;
    L.pv[s] = (int16_t)p;
  }
  lds_fence();
#pragma unroll
  for (int r = 0; r < WIDE_ROWS; ++r) {
    if (r >= rows) break;
    const int s = r * 64 + lane;
    uint32_t k = RANK_INF, m = 0;
    const int n = L.nx[s];
    if (((live[r] >> lane) & 1) && n >= 0) {
      const uint64_t v = wide_pair(t, w, a, L, s, n);
      if (v != ~0ULL) { k = (uint32_t)(v >> 32); m = (uint32_t)v; }
    }
    L.rk[s] = k;
    L.mid[s] = m;
  }
  uint32_t nfirst = 0, nlast = 0;
  for (;;) {
    lds_fence();
    uint32_t best = RANK_INF;
#pragma unroll
    for (int r = 0; r < WIDE_ROWS; ++r) {
      if (r >= rows) break;
      const int s = r * 64 + lane;
      const uint32_t k = L.rk[s];
      if (((live[r] >> lane) & 1) && k != RANK_INF) best = min(best, (k << 9) | (uint32_t)s);
    }
    best = wave_min_u32(best);
    if (best == RANK_INF) break;
    const uint32_t R = best >> 9;
    const int s0 = (int)(best & 511);
    uint64_t sel[WIDE_ROWS];
    if (rank_unsafe(t, R)) {
#pragma unroll
      for (int r = 0; r < WIDE_ROWS; ++r) sel[r] = (r == (s0 >> 6)) ? (1ULL << (s0 & 63)) : 0;
    } else {
      // leftmost non-overlapping occurrences, left to right
      int blocked = -1;
#pragma unroll
      for (int r = 0; r < WIDE_ROWS; ++r) {
        sel[r] = 0;
        if (r >= rows) continue;
        const int s = r * 64 + lane;
        uint64_t occ = __ballot(((live[r] >> lane) & 1) && L.rk[s] == R);
        while (occ) {
          const int b = __builtin_ctzll(occ);
          occ &= occ - 1;
          const int q = r * 64 + b;
          if (q != blocked) {
            sel[r] |= 1ULL << b;
            blocked = L.nx[q];
          }
        }
      }
    }
    if (hist) {
      // first live slot and last live slot of the piece
      int f = -1, l = -1;
      for (int r = 0; r < rows; ++r)
        if (live[r]) { f = r * 64 + __builtin_ctzll(live[r]); break; }
      for (int r = rows - 1; r >= 0; --r)
        if (live[r]) { l = r * 64 + 63 - __builtin_clzll(live[r]); break; }
      const int pl = L.pv[l];
      const bool fsel = (sel[f >> 6] >> (f & 63)) & 1;
      const bool lsel = pl >= 0 && ((sel[pl >> 6] >> (pl & 63)) & 1);
      if (t.cert == 2) {
        // the round: its rank, the product (one rule, so one id), and
        // whether it took the first / last token
        if (lane == 0)
          w.hfirst[a + nfirst] = ((uint64_t)R << 32) | (fsel ? HR_FIRST : 0) |
                                 (lsel ? HR_LAST : 0) | L.mid[s0];
        ++nfirst;
      } else {
        if (fsel) {
          if (lane == 0) w.hfirst[a + nfirst] = ((uint64_t)R << 32) | L.mid[f];
          ++nfirst;
        }
        if (lsel) {
          if (lane == 0) w.hlast[a + nlast] = ((uint64_t)R << 32) | L.mid[pl];
          ++nlast;
        }
      }
    }
    // a slot dies when its left neighbour is a selected left symbol
    uint64_t dead[WIDE_ROWS];
#pragma unroll
    for (int r = 0; r < WIDE_ROWS; ++r) {
      bool dies = false;
      if (r < rows) {
        const int s = r * 64 + lane;
        const int p = L.pv[s];
        dies = ((live[r] >> lane) & 1) && p >= 0 && ((sel[p >> 6] >> (p & 63)) & 1);
      }
      dead[r] = __ballot(dies);
    }
    lds_fence();
#pragma unroll
    for (int r = 0; r < WIDE_ROWS; ++r) {
      if (r >= rows) break;
      const int s = r * 64 + lane;
      if ((sel[r] >> lane) & 1) {
        const int rn = L.nx[s];
        const int nn = L.nx[rn];
        L.sym[s] = L.mid[s];
        L.nx[s] = (int16_t)nn;
        if (nn >= 0) L.pv[nn] = (int16_t)s;
      }
    }
#pragma unroll
    for (int r = 0; r < WIDE_ROWS; ++r) live[r] &= ~dead[r];
    lds_fence();
    // pairs that changed: the selected slots and the slots right before them
#pragma unroll
    for (int r = 0; r < WIDE_ROWS; ++r) {
      if (r >= rows) break;
      const int s = r * 64 + lane;
      if (!((live[r] >> lane) & 1)) continue;
      const int n = L.nx[s];
      const bool dirty = ((sel[r] >> lane) & 1) ||
                         (n >= 0 && ((sel[n >> 6] >> (n & 63)) & 1));
      if (!dirty) continue;
      uint32_t k = RANK_INF, m = 0;
      if (n >= 0) {
        const uint64_t v = wide_pair(t, w, a, L, s, n);
        if (v != ~0ULL) { k = (uint32_t)(v >> 32); m = (uint32_t)v; }
      }
      L.rk[s] = k;
      L.mid[s] = m;
    }
  }
  lds_fence();
#pragma unroll
  for (int r = 0; r < WIDE_ROWS; ++r) {
    if (r >= rows) break;
    const int s = r * 64 + lane;
    if (s < len)
      w.tok[a + s] = ((live[r] >> lane) & 1) ? (L.sym[s] & ~SYM_RAW) : INVALID_ID;
  }
  if (hist && lane == 0)
    w.hmeta[a] = t.cert == 2 ? nfirst : nfirst | (nlast << 16);
}

// Wave-wide minimum (the prefix minimum's last lane), as a scalar.
__device__ __forceinline__ uint32_t wave_min_dpp(uint32_t v) {
  v = dpp_min<0x111, 0xF>(v);
  v = dpp_min<0x112, 0xF>(v);
  v = dpp_min<0x114, 0xF>(v);
  v = dpp_min<0x118, 0xF>(v);
  v = dpp_min<0x142, 0xA>(v);
  v = dpp_min<0x143, 0xC>(v);
  return __builtin_amdgcn_readlane(v, 63);
}

// 64R-bit masks over a piece's positions, word r holding positions 64r ..
// 64r + 63 (wave-uniform, on the scalar unit). next_live_mask: for each
// bit q of `from`, the first live position after q, found as wave_bpe does
// on one word: a carry entered above q runs over the dead positions and
// stops on the first live one, (~live + (from << 1)) & live, with the
// carry passed from word to word. prev_live_mask: the last live position
// before each, the same on the bit-reversed masks.
template <int R>
__device__ __forceinline__ void next_live_mask(const uint64_t* live,
                                               const uint64_t* from,
                                               uint64_t* out) {
  unsigned long long c = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint64_t sh = (from[r] << 1) | (r ? from[r - 1] >> 63 : 0);
    unsigned long long co;
    const uint64_t s = __builtin_addcll(~live[r], sh, c, &co);
    out[r] = s & live[r];
    c = co;
  }
}

template <int R>
__device__ __forceinline__ void prev_live_mask(const uint64_t* live,
                                               const uint64_t* from,
                                               uint64_t* out) {
  uint64_t rl[R], rf[R], ro[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    rl[r] = __brevll(live[R - 1 - r]);
    rf[r] = __brevll(from[R - 1 - r]);
  }
  next_live_mask<R>(rl, rf, ro);
#pragma unroll
  for (int r = 0; r < R; ++r) out[r] = __brevll(ro[R - 1 - r]);
}

// One piece of 65..64R bytes merged by one wave with its state in registers:
// position p = 64r + lane sits in row r (symbol, pair rank and product per
// row and lane; live masks per row). Same order as wave_bpe_wide: each round
// takes the lowest-ranked pair, and a safe rank merges all its leftmost
// non-overlapping occurrences at once, an unsafe one its leftmost alone.
// Per round: one wave minimum, the selection on the scalar unit, and pair
// lookups for the positions whose pair changed (the winners and the live
// positions before them). H: the piece is a segment of a certified long
// piece, and its merge rounds go to the histories as wave_bpe_wide writes
// them (the repair passes' segments of 65..64R bytes).
template <int R, bool H>
__device__ __forceinline__ void wave_bpe_rows(const DevTables& t,
                                              const DevWork& w, uint32_t a,
                                              int len, bool vocab_first,
                                              const uint32_t* unsafe_lds,
                                              const uint4* hot) {
  const int lane = threadIdx.x & 63;
  if (vocab_first && t.ignore_merges) {
    int32_t hit = -1;
    if (lane == 0) hit = vocab_lookup(t, w.text + a, len);
    hit = __shfl(hit, 0);
    if (hit >= 0) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int p = 64 * r + lane;
        if (p < len) w.tok[a + p] = p == 0 ? (uint32_t)hit : INVALID_ID;
      }
      return;
    }
  }
  uint32_t sym[R], rk[R], mid[R];
  uint64_t live[R], dirty[R];
  uint32_t nfirst = 0, nlast = 0;  // (H) history entries written
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int p = 64 * r + lane;
    const uint32_t byte = p < len ? w.text[a + p] : 0u;
    const int32_t bid = p < len ? t.byte_id[byte] : -1;
    sym[r] = (uint32_t)bid | (byte << 20) | SYM_BYTE;
    live[r] = __ballot(bid >= 0);
    dirty[r] = live[r];
    rk[r] = RANK_INF;
    mid[r] = 0;
  }
  const uint64_t above = ~mask_le(lane);
  // next live position after position q (scalar), -1 when none
  auto next_live = [&](int q) {
    int res = -1;
#pragma unroll
    for (int r = R - 1; r >= 0; --r) {
      uint64_t m = live[r];
      if (r == (q >> 6)) m &= ~mask_le(q & 63);
      else if (r < (q >> 6)) m = 0;
      if (m) res = 64 * r + __builtin_ctzll(m);
    }
    return res;
  };
  for (;;) {
    // the first live position after each row
    int nf[R];
    {
      int f = -1;
#pragma unroll
      for (int r = R - 1; r >= 0; --r) {
        nf[r] = f;
        if (live[r]) f = 64 * r + __builtin_ctzll(live[r]);
      }
    }
    // pair ranks at the dirty positions
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (!dirty[r]) continue;  // wave-uniform
      const uint64_t after = live[r] & above;
      const int nl = after ? __builtin_ctzll(after) : 64;
      uint32_t ns = (uint32_t)__builtin_amdgcn_ds_bpermute(nl << 2, (int)sym[r]);
      bool has = nl < 64;
      if (nf[r] >= 0) {  // wave-uniform: the later rows' first live symbol
        uint32_t fs = 0;
#pragma unroll
        for (int q = r + 1; q < R; ++q)
          if ((nf[r] >> 6) == q) fs = __builtin_amdgcn_readlane(sym[q], nf[r] & 63);
        if (!has) ns = fs;
        has = true;
      }
      if (lane_bit(dirty[r])) {
        rk[r] = RANK_INF;
        if (has) {
          if (sym[r] & ns & SYM_BYTE) {
            const uint64_t v =
                t.bytepair[((sym[r] >> 12) & 0xFF00) | ((ns >> 20) & 0xFF)];
            if (v != ~0ULL) { rk[r] = (uint32_t)(v >> 32); mid[r] = (uint32_t)v; }
          } else if (t.ctab) {
            uint32_t r_, m_;
            if ((hot && hot_find(hot, t.hot_k, sym[r] & SYM_ID, ns & SYM_ID, &r_, &m_)) ||
                ctab_find(t, sym[r] & SYM_ID, ns & SYM_ID, &r_, &m_)) {
              rk[r] = r_;
              mid[r] = m_;
            }
          } else {
            const uint64_t v = pair_lookup(t, sym[r] & SYM_ID, ns & SYM_ID);
            if (v != ~0ULL) { rk[r] = (uint32_t)(v >> 32); mid[r] = (uint32_t)v; }
          }
        }
      }
    }
    uint32_t m = RANK_INF;
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (lane_bit(live[r]) && rk[r] != RANK_INF)
        m = min(m, (rk[r] << 9) | (uint32_t)(64 * r + lane));
    const uint32_t best = wave_min_dpp(m);
    if (best == RANK_INF) break;
    const uint32_t rank = best >> 9;
    const bool unsafe =
        unsafe_lds ? ((rank >> 5) < t.unsafe_words &&
                      ((unsafe_lds[rank >> 5] >> (rank & 31)) & 1))
                   : rank_unsafe(t, rank);
    // The round's merges as 64R-bit masks over the positions (word r: row
    // r): the pairs of this rank (occ), the winners (win), the positions
    // they absorb (gone: each winner's next live position) and the live
    // positions before them (prev), whose right neighbour changes.
    uint64_t occ[R], win[R], gone[R], prev[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
      occ[r] = __builtin_amdgcn_ballot_w64(lane_bit(live[r]) && rk[r] == rank);
    if (unsafe) {
      // an unsafe rank merges its leftmost pair alone
      bool found = false;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        win[r] = found ? 0 : occ[r] & (~occ[r] + 1);
        found = found || occ[r];
      }
    } else {
      // every pair of the rank, unless one's right symbol is the next
      // one's left: then leftmost first, each blocking the next
      next_live_mask<R>(live, occ, gone);
      uint64_t clash = 0;
#pragma unroll
      for (int r = 0; r < R; ++r) clash |= gone[r] & occ[r];
      if (!clash) {
#pragma unroll
        for (int r = 0; r < R; ++r) win[r] = occ[r];
      } else {
        int blocked = -1;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          win[r] = 0;
          uint64_t o = occ[r];
          while (o) {  // wave-uniform, positions in order
            const int q = 64 * r + __builtin_ctzll(o);
            o &= o - 1;
            if (q != blocked) {
              win[r] |= 1ULL << (q & 63);
              blocked = next_live(q);
            }
          }
        }
      }
    }
    if constexpr (H) {
      // the first live position f, the last one l and the live position
      // pl before it (the left symbol of the segment's last pair), all
      // wave-uniform; the round takes the first / last token when it
      // merges at f / pl
      int f = -1, l = -1, pl = -1;
#pragma unroll
      for (int r = R - 1; r >= 0; --r)
        if (live[r]) f = 64 * r + __builtin_ctzll(live[r]);
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (live[r]) l = 64 * r + 63 - __builtin_clzll(live[r]);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        uint64_t m = live[r];
        if (r == (l >> 6)) m &= (1ULL << (l & 63)) - 1;
        else if (r > (l >> 6)) m = 0;
        if (m) pl = 64 * r + 63 - __builtin_clzll(m);
      }
      auto won = [&](int q) {
        bool b = false;
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (r == (q >> 6)) b = (win[r] >> (q & 63)) & 1;
        return b;
      };
      auto product = [&](int q) {  // the pair product at position q
        uint32_t v = 0;
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (r == (q >> 6)) v = (uint32_t)__builtin_amdgcn_readlane((int)mid[r], q & 63);
        return v;
      };
      const bool fsel = won(f);
      const bool lsel = pl >= 0 && won(pl);
      if (t.cert == 2) {
        if (lane == 0)
          w.hfirst[a + nfirst] = ((uint64_t)rank << 32) | (fsel ? HR_FIRST : 0) |
                                 (lsel ? HR_LAST : 0) | product((int)(best & 511));
        ++nfirst;
      } else {
        if (fsel) {
          if (lane == 0) w.hfirst[a + nfirst] = ((uint64_t)rank << 32) | product(f);
          ++nfirst;
        }
        if (lsel) {
          if (lane == 0) w.hlast[a + nlast] = ((uint64_t)rank << 32) | product(pl);
          ++nlast;
        }
      }
    }
    next_live_mask<R>(live, win, gone);
    prev_live_mask<R>(live, win, prev);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (lane_bit(win[r])) sym[r] = mid[r];
      live[r] &= ~gone[r];
      dirty[r] = (win[r] | prev[r]) & live[r];
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int p = 64 * r + lane;
    if (p < len) w.tok[a + p] = lane_bit(live[r]) ? (sym[r] & SYM_ID) : INVALID_ID;
  }
  if (H && lane == 0) w.hmeta[a] = t.cert == 2 ? nfirst : nfirst | (nlast << 16);
}

// Entries of 65..WIDE_MAX bytes from a (start, end) list, one wave each.
__global__ __launch_bounds__(256) void k_bpe_wide(DevTables t, DevWork w,
                                                  const uint32_t* list,
                                                  const uint32_t* count,
                                                  uint32_t cap, int hist) {
  __shared__ WideLds lds[4];
  if (!pass_live(w)) return;
  uint32_t n = *count;
  if (n > cap) n = cap;
  const int wv = wave_id();
  const uint32_t waves = gridDim.x * 4;
  // With histories these are the segments of the certified long pieces,
  // one merge round after another on the request's critical path (the
  // cut / segment / certify chain ends last on C5): they get issue
  // priority over the other side work.
  if (hist && blockIdx.x * 4 + wv < n) __builtin_amdgcn_s_setprio(3);
  for (uint32_t k = blockIdx.x * 4 + wv; k < n; k += waves) {
    const uint32_t a = list[2 * k], b = list[2 * k + 1];
    const int len = (int)(b - a);
    // (pieces of up to 256 bytes without histories: k_bpe_pack, k_bpe_rows)
    if (len <= (hist ? 64 : 256) || len > WIDE_MAX) continue;  // wave-uniform
    wave_bpe_wide(t, w, a, len, !hist, hist != 0, lds[wv]);
  }
}

// Long-queue entries of 129..256 bytes, one wave each, state in registers
// (those of 65..128 bytes were merged by k_bpe_pack). With an unsafe-rank
// bitmap of at most ROWS_UNSAFE_LDS words, the launch gives each block a
// copy of it in LDS (one lookup per merge round).
constexpr uint32_t ROWS_UNSAFE_LDS = 12288;
__global__ __launch_bounds__(256) void k_bpe_rows(DevTables t, DevWork w) {
  extern __shared__ __align__(16) uint32_t unsafe_lds[];
  uint32_t n = *w.longcount;
  if (n > w.long_cap) n = w.long_cap;
  const bool lds = t.unsafe && t.unsafe_words <= ROWS_UNSAFE_LDS;
  if (lds)
    for (uint32_t j = threadIdx.x; j < t.unsafe_words; j += 256)
      unsafe_lds[j] = t.unsafe[j];
  // the hot-pair table after the bitmap (16-byte aligned)
  uint4* hot = nullptr;
  if (t.hot) {
    hot = reinterpret_cast<uint4*>(unsafe_lds + (lds ? (t.unsafe_words + 3) & ~3u : 0u));
    hot_stage(t, hot);
  }
  if (lds || hot) __syncthreads();
  const int lane = threadIdx.x & 63, wv = wave_id();
  // (no issue priority: the cut / segment / certify chain of the long
  // pieces takes it)
  // (pieces of 65..128 bytes too when k_bpe_pack left them: more than
  // PACK_ROWS_MAX queued)
  const int lo = n > (uint32_t)PACK_ROWS_MAX ? 64 : 128;
  // The queue in X contiguous shares (X = PACK_XCDS, or the blocks when
  // fewer), share x to the blocks of residue x (the blocks go to the XCDs
  // in turn). Wave g of a share's G waves takes entry g first, every later
  // one from the share's counter (G plus the count so far; the counters
  // start at 0 in each call's control slot), one at a time as waves finish
  // theirs: the waves end together instead of each on a fixed share whose
  // pieces' lengths it happened to draw.
  const uint32_t X = gridDim.x < (uint32_t)PACK_XCDS ? gridDim.x : (uint32_t)PACK_XCDS;
  const uint32_t x = blockIdx.x % X;
  const uint32_t k0 = (uint32_t)((uint64_t)n * x / X);
  const uint32_t k1 = (uint32_t)((uint64_t)n * (x + 1) / X);
  const uint32_t G = (gridDim.x - x + X - 1) / X * 4;
  uint32_t k = k0 + blockIdx.x / X * 4 + wv;
  while (k < k1) {
    const uint32_t a = w.longlist[2 * k], b = w.longlist[2 * k + 1];
    const int len = (int)(b - a);
    if (len > lo && len <= 256) {  // wave-uniform
      if (len <= 128) wave_bpe_rows<2>(t, w, a, len, true, lds ? unsafe_lds : nullptr, hot);
      else wave_bpe_rows<4>(t, w, a, len, true, lds ? unsafe_lds : nullptr, hot);
    }
    uint32_t got = 0;
    if (lane == 0)
      got = __hip_atomic_fetch_add(w.rowq + x, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    k = k0 + G + (uint32_t)__builtin_amdgcn_readfirstlane((int)got);
  }
}

__device__ __forceinline__ uint64_t inlong_window(const DevWork& w, int64_t v,
                                                  int phase) {
  if (phase == 0) return w.inlong[v];
  const uint64_t lo = v > 0 ? w.inlong[v - 1] : 0;
  return (lo >> 32) | (w.inlong[v] << 32);
}

// The grid windows that hold long-piece bytes (v in 0..nwin with a phase
// whose inlong_window is not empty), listed once each in vlist (vcount of
// them), in no particular order. The window, segment and certify kernels
// keep a wave per window of the text, but wave i takes listed window i:
// the waves with work are the grid's first (on C5 ten runs fill ~20,000 of
// ~150,000 windows, spread through the text, and the waves for them came
// between the empty ones), and the rest end at once. (A fixed grid of
// 1024 or 2048 blocks walking the list from a counter was slower: C5
// 1.92 / 2.01 ms against 1.82; this order: 1.73.)
__global__ void k_win_list(DevWork w, int64_t nwin) {
  const int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  bool need = false;
  if (v <= nwin)
    for (int phase = (v == nwin ? 1 : 0); phase < 2; ++phase)
      need = need || inlong_window(w, v, phase) != 0;
  const uint64_t m = __ballot(need);
  if (!m) return;
  const int lane = threadIdx.x & 63;
  uint32_t base = 0;
  if (lane == 0) base = atomicAdd(w.vcount, (uint32_t)__popcll(m));
  base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
  if (need) w.vlist[base + (uint32_t)__popcll(m & ((1ULL << lane) - 1))] = (uint32_t)v;
}

__device__ __forceinline__ void long_window(const DevTables& t, const DevWork& w,
                                            int64_t v, int64_t nwin) {
  const int lane = threadIdx.x & 63;
  auto seg = [&](int64_t wd) { return w.starts[wd]; };
  uint16_t* cut16 = reinterpret_cast<uint16_t*>(w.cuts);
  for (int phase = (v == nwin ? 1 : 0); phase < 2; ++phase) {
    const uint64_t L = inlong_window(w, v, phase);
    if (L == 0) continue;  // wave-uniform
    const int64_t base = phase == 0 ? v * 64 : v * 64 - 32;
    uint64_t S;
    bool E;
    window_bits(v, phase, seg, &S, &E);
    S |= 1;  // the window start cuts whatever runs into it
    const uint64_t le = S & mask_le(lane);
    const int ps = 63 - __builtin_clzll(le);
    const uint64_t gt = S & ~mask_le(lane);
    const int pe = gt ? __builtin_ctzll(gt) : 64;
    const bool elig = (L >> lane) & 1;
    const uint64_t live =
        wave_bpe<false, false, false>(t, w, base, base + lane, lane, elig, ps, pe);
    if (lane == 0) {
      if (phase == 0) {
        cut16[4 * v + 1] = (uint16_t)(live >> 16);
        cut16[4 * v + 2] = (uint16_t)(live >> 32);
      } else {
        if (v > 0) cut16[4 * (v - 1) + 3] = (uint16_t)(live >> 16);
        cut16[4 * v] = (uint16_t)(live >> 32);
      }
    }
  }
}

// Cut selection: BPE of the long-piece bytes of every window, window edges
// taken as cuts; the token starts in the window's central 32 bytes become
// candidate cuts. Aligned window v owns bits 16..47 of word v, shifted
// window v owns bits 48..63 of word v-1 and 0..15 of word v. Wave i takes
// listed window i.
__global__ __launch_bounds__(256) void k_long_windows(DevTables t, DevWork w,
                                                      int64_t nwin) {
  const uint32_t i = blockIdx.x * 4 + wave_id();
  if (i >= *w.vcount) return;
  // the long pieces' chain (windows, segments, certification, repairs)
  // sets the end of a request that has any: issue priority
  __builtin_amdgcn_s_setprio(2);
  long_window(t, w, w.vlist[i], nwin);
}

__device__ __forceinline__ uint64_t seg_word(const DevWork& w, int64_t wd) {
  return w.starts[wd] | (w.cuts[wd] & w.inlong[wd]);
}

__device__ __forceinline__ bool word_dirty(const uint64_t* d, int64_t wd) {
  return wd >= 0 && ((d[wd >> 6] >> (wd & 63)) & 1);
}

// A first-pass segment [a, b) over 64 bytes (a stretch with few cut
// candidates): instead of merging it on this pass, beside the row merges,
// with a kernel that needs LDS or 1024-thread blocks (no room for either
// until the row merges end: 200-400 us of C5's critical path), its
// bounding cuts are failed as certification fails a cut, so the first
// repair pass joins it to its neighbours and merges the joined segment
// (k_seg_scan lists it from its dirty words; k_repair_merge, k_seg_block).
// Dropping a cut is always safe: the cuts that remain are certified. One
// lane.
__device__ void fail_segment_cuts(const DevWork& w, int64_t a, int64_t b) {
  auto is_cut = [&](int64_t c) {
    const int64_t wd = c >> 6;
    return ((w.cuts[wd] & w.inlong[wd] & ~w.starts[wd]) >> (c & 63)) & 1;
  };
  auto fail = [&](int64_t c) {
    atomicOr(reinterpret_cast<unsigned long long*>(&w.failm[c >> 6]), 1ULL << (c & 63));
    atomicAdd(w.nfail, 1u);
  };
  int64_t lo = a, hi = b;
  // (a segment bounded by piece starts alone still counts one failure, so
  // that the repair pass runs and lists it)
  if (!is_cut(a) && !is_cut(b)) atomicAdd(w.nfail, 1u);
  if (is_cut(a)) {
    fail(a);
    // start of the segment that ends at a
    int64_t wd = a >> 6;
    uint64_t word = seg_word(w, wd) & ((1ULL << (a & 63)) - 1);
    while (word == 0) word = seg_word(w, --wd);
    lo = wd * 64 + (63 - __builtin_clzll(word));
  }
  if (is_cut(b)) {
    fail(b);
    // end of the segment that starts at b
    int64_t we = b >> 6;
    uint64_t up = seg_word(w, we) & ~mask_le((int)(b & 63));
    while (up == 0) up = seg_word(w, ++we);
    hi = we * 64 + __builtin_ctzll(up);
  }
  for (int64_t q = lo >> 6; q <= (hi >> 6); ++q)
    atomicOr(reinterpret_cast<unsigned long long*>(&w.dirty_next[q >> 6]),
             1ULL << (q & 63));
}

// Segment work of one grid window (phase 0: aligned [64v, 64v+64), phase 1:
// shifted [64v-32, 64v+32)): the BPE of the long-piece segments the window
// holds whole, with histories. With `push`, phase 0 also lists the segment
// that starts in the window and fits no grid window (seglist). Wave-uniform.
__device__ __forceinline__ void segment_window(const DevTables& t, const DevWork& w,
                                               int64_t v, int phase, bool push) {
  const int lane = threadIdx.x & 63;
  auto seg = [&](int64_t wd) { return seg_word(w, wd); };
  const uint64_t L = inlong_window(w, v, phase);
  if (L == 0) return;
  const int64_t base = phase == 0 ? v * 64 : v * 64 - 32;
  uint64_t S;
  bool E;
  window_bits(v, phase, seg, &S, &E);
  const int64_t pos = base + lane;
  const bool inl = (L >> lane) & 1;
  const uint64_t le = S & mask_le(lane);
  const int ps = le ? 63 - __builtin_clzll(le) : -1;
  const uint64_t gt = S & ~mask_le(lane);
  const int pe = gt ? __builtin_ctzll(gt) : 64;
  const bool contained = ps >= 0 && (pe < 64 || E);
  bool elig = inl && contained;
  if (phase == 1 && elig && ((base + ps) >> 6) == ((base + pe - 1) >> 6))
    elig = false;
  if (push && phase == 0 && inl && ps == lane && !contained) {
    const int64_t b = seg_end_after(v + 1, seg);
    if (!fits_a_grid(pos, b)) {
      if (b - pos > 64) fail_segment_cuts(w, pos, b);
      else push_pair(w.seglist, w.segcount, w.seg_cap, w.status, pos, b);
    }
  }
  wave_bpe<false, true, true>(t, w, base, base + lane, lane, elig, ps, pe);
}

// Segment pass over the long-piece bytes (64-byte grid windows, aligned and
// shifted by 32, with histories), wave i over listed window i. Segments
// that fit no grid window go to seglist. (The
// repair passes redo only the windows of dirty words: k_seg_scan,
// k_repair_merge.)
__global__ __launch_bounds__(256) void k_long_segments(DevTables t, DevWork w,
                                                       int64_t nwin) {
  const uint32_t i = blockIdx.x * 4 + wave_id();
  if (i >= *w.vcount || !pass_live(w)) return;
  __builtin_amdgcn_s_setprio(2);  // (the long pieces' chain: k_long_windows)
  const int64_t v = w.vlist[i];
  for (int phase = (v == nwin ? 1 : 0); phase < 2; ++phase)
    segment_window(t, w, v, phase, true);
}

// A repair pass's work list, one thread per text word d: when d is dirty,
// every window k_long_segments would redo for it (v = d: both phases; v =
// d + 1 when that word is not dirty itself: phase 1), as v << 1 | (phase 0
// too), and the segment it would list (the segment that starts at d's last
// start, runs past d and fits no grid window). Run after k_apply_fail, so
// the cuts are final for the pass. (One thread per 64 words walked a
// pass's thousands of dirty words 64 at a time: 34 us on C5's first pass.)
__global__ void k_seg_scan(DevWork w, int64_t nwin) {
  const int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (d > nwin || !pass_live(w)) return;
  if (!word_dirty(w.dirty_cur, d)) return;
  auto seg = [&](int64_t wd) { return seg_word(w, wd); };
  auto put = [&](uint32_t item) {
    const uint32_t k = atomicAdd(w.wcount, 1u);
    if (k < w.wlist_cap) w.wlist[k] = item;
    else atomicOr(w.status, ST_LONGOVF);
  };
  put(((uint32_t)d << 1) | (d < nwin ? 1u : 0u));
  if (d + 1 <= nwin && !word_dirty(w.dirty_cur, d + 1)) put((uint32_t)(d + 1) << 1);
  if (d < nwin) {
    const uint64_t S = seg(d);
    if (S) {
      const int st = 63 - __builtin_clzll(S);  // the word's last start
      if (((w.inlong[d] >> st) & 1) && !(seg(d + 1) & 1)) {
        const int64_t a = 64 * d + st;
        const int64_t b = seg_end_after(d + 1, seg);
        if (!fits_a_grid(a, b))
          push_pair(w.seglist, w.segcount, w.seg_cap, w.status, a, b);
      }
    }
  }
}

// The first pass's listed segments (each at most 64 bytes: the longer ones
// had their cuts failed), one wave each, with histories. No LDS and few
// registers, so its waves find room beside the row merges (whose LDS holds
// the unsafe-rank bitmap on tables that have one).
__global__ __launch_bounds__(256) void k_seg_short(DevTables t, DevWork w) {
  const int lane = threadIdx.x & 63;
  if (!pass_live(w)) return;
  uint32_t n = *w.segcount;
  if (n > w.seg_cap) n = w.seg_cap;
  const uint32_t waves = gridDim.x * 4;
  const uint32_t k0 = blockIdx.x * 4 + wave_id();
  // (the long pieces' chain, as k_repair_merge)
  if (k0 < n) __builtin_amdgcn_s_setprio(3);
  for (uint32_t k = k0; k < n; k += waves) {
    const uint32_t a = w.seglist[2 * k], b = w.seglist[2 * k + 1];
    const int len = (int)(b - a);
    if (len > 64) {  // (not listed on this pass; an internal error if seen)
      if (lane == 0) atomicOr(w.status, ST_ROUNDS);
      continue;
    }
    wave_bpe<false, true, true>(t, w, (int64_t)a, (int64_t)a + lane, lane, lane < len, 0, len);
  }
}

// A repair pass's merges in one launch: the listed segments of up to
// WIDE_MAX bytes (first: the longest chains) and the listed windows, one
// wave per entry, all at once (in separate launches they ran one after the
// other, each as long as its slowest wave).
__global__ __launch_bounds__(256) void k_repair_merge(DevTables t, DevWork w,
                                                      int64_t nwin) {
  __shared__ WideLds lds[4];
  if (!pass_live(w)) return;
  uint32_t ns = *w.segcount;
  if (ns > w.seg_cap) ns = w.seg_cap;
  uint32_t nw = *w.wcount;
  if (nw > w.wlist_cap) nw = w.wlist_cap;
  const int lane = threadIdx.x & 63;
  const int wv = wave_id();
  const uint32_t waves = gridDim.x * 4;
  // (the long pieces' chain, as k_bpe_wide's segments with histories)
  if (blockIdx.x * 4 + wv < ns + nw) __builtin_amdgcn_s_setprio(3);
  for (uint32_t k = blockIdx.x * 4 + wv; k < ns + nw; k += waves) {
    if (k < ns) {
      const uint32_t a = w.seglist[2 * k], b = w.seglist[2 * k + 1];
      const int len = (int)(b - a);
      if (len <= 64)
        wave_bpe<false, true, true>(t, w, (int64_t)a, (int64_t)a + lane, lane,
                                    lane < len, 0, len);
      else if (len <= 128)  // (state in registers: about half the LDS
        // merge's time per round)
        wave_bpe_rows<2, true>(t, w, a, len, false, nullptr);
      else if (len <= 256)
        wave_bpe_rows<4, true>(t, w, a, len, false, nullptr);
      else if (len <= WIDE_MAX)
        wave_bpe_wide(t, w, a, len, false, true, lds[wv]);
    } else {
      const uint32_t it = w.wlist[k - ns];
      const int64_t v = (int64_t)(it >> 1);
      if (it & 1) segment_window(t, w, v, 0, false);
      segment_window(t, w, v, 1, false);
    }
  }
}

// Segments (mode 0: seglist, with histories) or whole pieces (mode 1:
// longlist, a whole-vocabulary entry first; tables that drop bytes) over
// WIDE_MAX bytes, one workgroup each: the block's threads look through the
// block's share of the list for them, then merge them one by one.
constexpr int SEGB_GRID = 128;
__global__ __launch_bounds__(SEGB_TPB) void k_seg_block(DevTables t, DevWork w,
                                                        const uint32_t* list,
                                                        const uint32_t* count,
                                                        uint32_t cap, int mode) {
  __shared__ SegLds L;
  if (mode == 0 && !pass_live(w)) return;
  uint32_t n = *count;
  if (n > cap) n = cap;
  for (uint32_t base = blockIdx.x * SEGB_TPB; base < n; base += gridDim.x * SEGB_TPB) {
    if (threadIdx.x == 0) L.nq = 0;
    __syncthreads();
    const uint32_t k = base + threadIdx.x;
    if (k < n && list[2 * k + 1] - list[2 * k] > (uint32_t)WIDE_MAX)
      L.queue[atomicAdd(&L.nq, 1u)] = k;
    __syncthreads();
    const uint32_t nq = L.nq;
    for (uint32_t j = 0; j < nq; ++j) {
      const uint32_t kk = L.queue[j];
      block_bpe(t, w, list[2 * kk], list[2 * kk + 1], mode == 1, mode == 0, L);
    }
    __syncthreads();
  }
}

// Certify every cut: one wave per bitmask word, one lane per cut (in a
// repair pass only the dirty words). A failing cut is recorded in failm and
// counted, and the words of the two segments it joins are marked dirty for
// the next pass.
__device__ __forceinline__ uint32_t pair_rank(const DevTables& t, uint32_t l,
                                              uint32_t r) {
  uint32_t rank, id;
  return pair_find(t, l, r, &rank, &id) ? rank : RANK_INF;
}

// A segment's history entries read in order, four loads ahead of the one
// in use: the walk below takes one entry per step, and each step's pair
// lookup no longer waits behind the load of the entry it needs.
struct EvStream {
  const uint64_t* e;
  uint32_t n, i;
  uint64_t q0, q1, q2, q3;
  __device__ __forceinline__ uint64_t at(uint32_t k) const {
    return k < n ? e[k] : ~0ULL;
  }
  __device__ __forceinline__ void init(const uint64_t* p, uint32_t cnt) {
    e = p;
    n = cnt;
    i = 0;
    q0 = at(0);
    q1 = at(1);
    q2 = at(2);
    q3 = at(3);
  }
  // the next entry's rank, RANK_INF past the last one
  __device__ __forceinline__ uint32_t rank() const {
    return i < n ? (uint32_t)(q0 >> 32) : RANK_INF;
  }
  __device__ __forceinline__ uint64_t take() {
    const uint64_t v = q0;
    q0 = q1;
    q1 = q2;
    q2 = q3;
    q3 = at(i + 4);
    ++i;
    return v;
  }
};

// One cut c = 64v + bit (the calling lane's).
__device__ void certify_cut(const DevTables& t, const DevWork& w, int64_t v, int bit) {
  const int64_t c = v * 64 + bit;
  // start of the segment that ends at c
  int64_t wd = v;
  uint64_t word = seg_word(w, wd) & ((1ULL << bit) - 1);
  while (word == 0) word = seg_word(w, --wd);
  const int64_t a = wd * 64 + (63 - __builtin_clzll(word));
  uint32_t L = (uint32_t)t.byte_id[w.text[c - 1]];
  uint32_t R = (uint32_t)t.byte_id[w.text[c]];
  bool ok = true;
  uint32_t rho = pair_rank(t, L, R);
  EvStream A, B;
  if (t.cert == 2) {
    // Any table: the two segments' merge rounds in the order the whole
    // piece would run them (the left segment's next round first when its
    // rank is at most the right one's: its pairs lie to the left), and at
    // every state the pair across c must lose to one of the two heads. A
    // round of several merges runs at a rank no earlier rule consumes the
    // product of, so the pair it leaves across c while it goes on ranks
    // above it and cannot merge then: the states between rounds are the
    // ones to check.
    A.init(w.hfirst + a, w.hmeta[a]);
    B.init(w.hfirst + c, w.hmeta[c]);
    for (;;) {
      const uint32_t ra = A.rank(), rb = B.rank();
      if (rho < ra && rho <= rb) { ok = false; break; }  // merges across c
      if (ra == RANK_INF && rb == RANK_INF) break;
      if (ra <= rb) {
        const uint64_t e = A.take();
        if (e & HR_LAST) {
          L = (uint32_t)e & SYM_ID;
          rho = pair_rank(t, L, R);
        }
      } else {
        const uint64_t e = B.take();
        if (e & HR_FIRST) {
          R = (uint32_t)e & SYM_ID;
          rho = pair_rank(t, L, R);
        }
      }
    }
  } else {
    A.init(w.hlast + a, w.hmeta[a] >> 16);
    B.init(w.hfirst + c, w.hmeta[c] & 0xFFFF);
    for (;;) {
      const uint32_t ra = A.rank(), rb = B.rank();
      if (rho < ra && rho <= rb) { ok = false; break; }  // merges across c
      if (ra == RANK_INF && rb == RANK_INF) break;
      if (ra <= rb) L = (uint32_t)A.take();
      if (rb <= ra) R = (uint32_t)B.take();
      rho = pair_rank(t, L, R);
    }
  }
  if (!ok) {
    atomicOr(reinterpret_cast<unsigned long long*>(&w.failm[v]), 1ULL << bit);
    atomicAdd(w.nfail, 1u);
    // end of the segment that starts at c
    int64_t we = v;
    uint64_t up = seg_word(w, we) & ~mask_le(bit);
    while (up == 0) up = seg_word(w, ++we);
    const int64_t e = we * 64 + __builtin_ctzll(up);
    for (int64_t q = a >> 6; q <= (e >> 6); ++q)
      atomicOr(reinterpret_cast<unsigned long long*>(&w.dirty_next[q >> 6]),
               1ULL << (q & 63));
  }
}

// Certify the cuts of the listed windows' words (a word holds cuts only
// where it holds long-piece bytes, so every such word is listed): wave i
// over listed word i (in a repair pass only the dirty words).
__global__ __launch_bounds__(256) void k_certify(DevTables t, DevWork w,
                                                 int64_t nwords, int all) {
  const int lane = threadIdx.x & 63;
  if (!pass_live(w)) return;
  const uint32_t i = blockIdx.x * 4 + wave_id();
  if (i >= *w.vcount) return;
  const int64_t v = w.vlist[i];
  if (v >= nwords) return;
  if (!all && !word_dirty(w.dirty_cur, v)) return;  // wave-uniform
  const uint64_t cuts = w.cuts[v] & w.inlong[v] & ~w.starts[v];
  if (!cuts) return;
  // (the long pieces' chain: the first pass runs beside the row merges)
  __builtin_amdgcn_s_setprio(2);
  if ((cuts >> lane) & 1) certify_cut(t, w, v, lane);
}

// Between passes: drop the failed cuts, and make the words marked by the
// last certify pass the dirty set of the next one. It starts a pass: its
// failed-cut count starts at zero (a pass that does not run leaves zero,
// so none after it runs either), and, when the pass runs, its segment list
// is emptied and the pass counted.
__global__ void k_apply_fail(DevWork w, int64_t nwords) {
  const int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = pass_live(w);
  if (v == 0) {
    *w.nfail = 0;
    if (live) {
      *w.segcount = 0;
      *w.wcount = 0;
      if (w.npass) *w.npass += 1;
    }
  }
  if (v >= nwords || !live) return;
  const uint64_t f = w.failm[v];
  if (f) {
    w.cuts[v] &= ~f;
    w.failm[v] = 0;
  }
  if (v < (nwords + 63) / 64 + 1) {
    w.dirty_cur[v] = w.dirty_next[v];
    w.dirty_next[v] = 0;
  }
}

// A widened repair pass (from the pass TK_OPT_REPAIR_WIDEN names on): a
// failed cut also drops the `width` nearest cuts on each side of it inside
// its piece. Without it a pass can expose the next failing cut each time:
// in a periodic run whose token parity its first window fixes ("!" +
// "QQQ...": every later window pairs the letters from an even offset),
// removing a failed cut makes the one after it fail, one cut per pass,
// 35,000 passes for 70,000 letters. The width grows fourfold a pass, so a
// cascade of L cuts ends in about log4(L) passes, while the isolated
// failures of ordinary text (all fixed by the third pass on C5) never see
// it. One thread per failed-cut word, ahead of k_apply_fail; the words
// from the new segment's start to its end are marked dirty for the pass.
// Clears by other threads only shorten what a thread sees, so it drops
// more, never less, and the union of the marked ranges covers every joined
// segment.
__global__ void k_fail_widen(DevWork w, int64_t nwords, uint32_t width) {
  const int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (v >= nwords || !pass_live(w)) return;
  uint64_t f = w.failm[v];
  while (f) {
    const int bit = __builtin_ctzll(f);
    f &= f - 1;
    const int64_t c = v * 64 + bit;
    auto drop = [&](int64_t wd, int b) {
      atomicAnd(reinterpret_cast<unsigned long long*>(&w.cuts[wd]), ~(1ULL << b));
    };
    // down: clear `width` cuts, stop at the piece start or the next cut
    int64_t lo = c;
    {
      uint32_t k = 0;
      int64_t wd = v;
      uint64_t m = bit ? (1ULL << bit) - 1 : 0;  // bits below c in its word
      for (;;) {
        const uint64_t st = w.starts[wd];
        uint64_t sb = (st | (w.cuts[wd] & w.inlong[wd])) & m;
        bool done = false;
        while (sb) {
          const int b = 63 - __builtin_clzll(sb);
          sb &= ~(1ULL << b);
          if (((st >> b) & 1) || k == width) {
            lo = wd * 64 + b;
            done = true;
            break;
          }
          drop(wd, b);
          ++k;
        }
        if (done || wd == 0) break;
        --wd;
        m = ~0ULL;
      }
    }
    // up: the same towards the piece end (a start bit; sentinel start bits
    // lie past the text)
    int64_t hi = c;
    {
      uint32_t k = 0;
      int64_t wd = v;
      uint64_t m = ~mask_le(bit);  // bits above c in its word
      for (;;) {
        const uint64_t st = w.starts[wd];
        uint64_t sb = (st | (w.cuts[wd] & w.inlong[wd])) & m;
        bool done = false;
        while (sb) {
          const int b = __builtin_ctzll(sb);
          sb &= sb - 1;
          if (((st >> b) & 1) || k == width) {
            hi = wd * 64 + b;
            done = true;
            break;
          }
          drop(wd, b);
          ++k;
        }
        if (done) break;
        ++wd;
        m = ~0ULL;
      }
    }
    for (int64_t q = lo >> 6; q <= (hi >> 6); ++q)
      atomicOr(reinterpret_cast<unsigned long long*>(&w.dirty_next[q >> 6]),
               1ULL << (q & 63));
  }
}

// Pieces of 129..256 bytes (k_bpe_rows) and of 257..WIDE_MAX bytes
// (k_bpe_wide, state in LDS) are merged whole, one wave each, once the host
// knows there are any (a wave per queued piece, up to 2048 blocks of four;
// those of 65..128 bytes were merged by k_bpe_pack).
// Its waves loop over the queue, so the grid is capped at half the
// machine's wave slots: with all of them (2048 blocks) the loop held every
// slot while the long pieces' window kernel ran, and that kernel, on C5's
// critical path, starved (846 us; 277 us with a quarter of the slots, but
// the row merge then took 2 ms).
constexpr uint32_t ROWS_MAX_BLOCKS = 1024;
hipError_t launch_bpe_rows(const DevTables& t, const DevWork& w, hipStream_t s,
                           uint32_t nlong, hipEvent_t start, hipEvent_t stop) {
  const uint32_t blocks = nlong / 4 + 1 < ROWS_MAX_BLOCKS ? nlong / 4 + 1 : ROWS_MAX_BLOCKS;
  size_t lds = t.unsafe && t.unsafe_words <= ROWS_UNSAFE_LDS
                   ? (size_t)((t.unsafe_words + 3) & ~3u) * 4 : 0;
  if (t.hot) lds += HOT_BYTES;
  if (start || stop)
    hipExtLaunchKernelGGL(k_bpe_rows, dim3(blocks), dim3(256), lds, s, start, stop,
                          0, t, w);
  else
    hipLaunchKernelGGL(k_bpe_rows, dim3(blocks), dim3(256), lds, s, t, w);
  return hipGetLastError();
}

hipError_t launch_bpe_wide(const DevTables& t, const DevWork& w, hipStream_t s,
                           hipEvent_t stop, uint32_t nlong) {
  const uint32_t blocks = nlong / 4 + 1 < 2048 ? nlong / 4 + 1 : 2048;
  launch_ev(k_bpe_wide, dim3(blocks), dim3(256), s, nullptr, stop, t, w,
            (const uint32_t*)w.longlist, (const uint32_t*)w.longcount,
            w.long_cap, 0);
  return hipGetLastError();
}

hipError_t launch_long_windows(const DevTables& t, const DevWork& w,
                               hipStream_t s, hipEvent_t start, hipEvent_t stop) {
  const int64_t nwin = (w.nb + 63) / 64;
  launch_ev(k_win_list, dim3((uint32_t)((nwin + 1 + 255) / 256)), dim3(256), s,
            start, nullptr, w, nwin);
  launch_ev(k_long_windows, dim3((uint32_t)((nwin + 4) / 4)), dim3(256), s, nullptr,
            stop, t, w, nwin);
  return hipGetLastError();
}

hipError_t launch_long_segments(const DevTables& t, const DevWork& w, hipStream_t s) {
  const int64_t nwin = (w.nb + 63) / 64;
  hipLaunchKernelGGL(k_long_segments, dim3((uint32_t)((nwin + 4) / 4)), dim3(256), 0,
                     s, t, w, nwin);
  return hipGetLastError();
}

// The first pass's listed segments (each at most 64 bytes: the longer ones
// had their cuts failed, fail_segment_cuts), one wave each (k_seg_short).
constexpr uint32_t REPAIR_BLOCKS = 512;
hipError_t launch_seg_lists(const DevTables& t, const DevWork& w, hipStream_t s) {
  hipLaunchKernelGGL(k_seg_short, dim3(1024), dim3(256), 0, s, t, w);
  return hipGetLastError();
}

hipError_t launch_repair_segments(const DevTables& t, const DevWork& w, hipStream_t s) {
  const int64_t nwin = (w.nb + 63) / 64;
  hipLaunchKernelGGL(k_seg_scan, dim3((uint32_t)((nwin + 1 + 255) / 256)), dim3(256),
                     0, s, w, nwin);
  hipLaunchKernelGGL(k_repair_merge, dim3(REPAIR_BLOCKS), dim3(256), 0, s, t, w, nwin);
  hipLaunchKernelGGL(k_seg_block, dim3(SEGB_GRID), dim3(SEGB_TPB), 0, s, t, w,
                     (const uint32_t*)w.seglist, (const uint32_t*)w.segcount,
                     w.seg_cap, 0);
  return hipGetLastError();
}

hipError_t launch_long_block(const DevTables& t, const DevWork& w, hipStream_t s) {
  hipLaunchKernelGGL(k_seg_block, dim3(SEGB_GRID), dim3(SEGB_TPB), 0, s, t, w,
                     (const uint32_t*)w.longlist, (const uint32_t*)w.longcount,
                     w.long_cap, 1);
  return hipGetLastError();
}

hipError_t launch_certify(const DevTables& t, const DevWork& w, int all,
                          hipStream_t s, hipEvent_t stop) {
  const int64_t nwords = (w.nb + 63) / 64;
  launch_ev(k_certify, dim3((uint32_t)((nwords + 4) / 4)), dim3(256), s, nullptr,
            stop, t, w, nwords, all);
  return hipGetLastError();
}

hipError_t launch_apply_fail(const DevWork& w, hipStream_t s, uint32_t width) {
  const int64_t nwords = (w.nb + 63) / 64;
  if (width)
    hipLaunchKernelGGL(k_fail_widen, dim3((uint32_t)((nwords + 255) / 256)),
                       dim3(256), 0, s, w, nwords, width);
  hipLaunchKernelGGL(k_apply_fail, dim3((uint32_t)((nwords + 255) / 256)),
                     dim3(256), 0, s, w, nwords);
  return hipGetLastError();
}

// ------------------------------------------------------ 4. compaction

// One pass over the token slots: every block counts the ids in its
// COMPACT_BLOCK slots (a wave per quarter, 64 consecutive slots a step) and
// stages them in LDS, publishes the count, takes its offset from its
// predecessors' words (decoupled look-back: the nearest predecessor that has
// published a running total, plus the counts in between, 64 * COMPACT_LOOK
// predecessors per step), publishes its running total and stores its ids
// contiguously. The status words are read past L2 (agent scope), so every
// word read costs a trip to the memory side for every block of the launch:
// a short window per step and large blocks keep those reads few.
// A status word is tag << 32 | CST_TOTAL (a running total, else a count) |
// value: words left by other launches carry other tags and read as not yet
// published. A block waits only for blocks dispatched before it, which
// publish their counts without waiting, and every wait is bounded.
constexpr uint32_t CST_TOTAL = 1u << 31;
constexpr int COMPACT_LOOK = 1;

__device__ __forceinline__ void cst_store(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t cst_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ __launch_bounds__(COMPACT_TPB) void k_compact(DevWork w, int64_t nblk,
                                                         uint32_t tag) {
  __shared__ uint32_t sbase;
  // the block's ids: wave g's, in position order, from sout[g * CW]
  constexpr int CW = COMPACT_BLOCK / (COMPACT_TPB / 64);
  __shared__ uint32_t sout[COMPACT_BLOCK];
  __shared__ uint32_t wcnt[COMPACT_TPB / 64];
  const int tid = threadIdx.x, lane = tid & 63, wv = wave_id();
  const int64_t b = blockIdx.x;
  // Wave g compacts the block's g-th CW positions, 64 a step (lane l reads
  // position 64k + l): the step's ids go to the next consecutive LDS words
  // at the ballot's prefix (neighbouring lanes, neighbouring banks).
  {
    const int64_t p0 = b * COMPACT_BLOCK + (int64_t)wv * CW + lane;
    const uint64_t below = (1ULL << lane) - 1;
    // every load first (one memory round trip), then the ballots
    uint32_t v[CW / 64];
    if (p0 - lane + CW <= w.nb) {  // wave-uniform: the whole quarter is text
#pragma unroll
      for (int k = 0; k < CW / 64; ++k) v[k] = w.tok[p0 + 64 * k];
    } else {
#pragma unroll
      for (int k = 0; k < CW / 64; ++k)
        v[k] = p0 + 64 * k < w.nb ? w.tok[p0 + 64 * k] : INVALID_ID;
    }
    uint32_t run = 0;
#pragma unroll
    for (int k = 0; k < CW / 64; ++k) {
      const uint64_t m = __ballot(v[k] != INVALID_ID);
      if (v[k] != INVALID_ID) sout[wv * CW + run + (uint32_t)__popcll(m & below)] = v[k];
      run += (uint32_t)__popcll(m);
    }
    if (lane == 0) wcnt[wv] = run;
  }
  __syncthreads();
  uint32_t pre[COMPACT_TPB / 64];  // the ids of the waves before each wave
  uint32_t tot = 0;
#pragma unroll
  for (int g = 0; g < COMPACT_TPB / 64; ++g) {
    pre[g] = tot;
    tot += wcnt[g];
  }
  if (wv == 0) {
    const uint64_t hi = (uint64_t)tag << 32;
    uint32_t base = 0;
    bool ok = true;
    if (b == 0) {
      if (lane == 0) cst_store(&w.cstat[0], hi | CST_TOTAL | tot);
    } else {
      if (lane == 0) cst_store(&w.cstat[b], hi | tot);
      // COMPACT_LOOK * 64 predecessors per step, nearest first: lane l of
      // part k reads block j - 64k - l (blocks before 0 read as a running
      // total of 0)
      for (int64_t j = b - 1;; j -= 64 * COMPACT_LOOK) {
        uint64_t st[COMPACT_LOOK];
#pragma unroll
        for (int k = 0; k < COMPACT_LOOK; ++k) {
          const int64_t q = j - 64 * k - lane;
          st[k] = q >= 0 ? cst_load(&w.cstat[q]) : (hi | CST_TOTAL);
        }
        // Only the words before the nearest published running total are
        // needed: wait for those (every unpublished one re-read at once,
        // one round trip per round), and never for the words behind it.
        for (WaitBound wb;;) {
          bool need = false, found = false;
#pragma unroll
          for (int k = 0; k < COMPACT_LOOK; ++k) {
            if (found) break;  // wave-uniform
            const bool pub = (st[k] >> 32) == tag;
            const uint64_t tm = __ballot(pub && ((uint32_t)st[k] & CST_TOTAL) != 0);
            const int l = tm ? __builtin_ctzll(tm) : 64;
            need |= __ballot(!pub && lane < l) != 0;
            found = tm != 0;
          }
          if (!need) break;
          if (wb.expired(w.wait_ticks)) {  // only after the bounded wait
            ok = false;
#pragma unroll
            for (int k = 0; k < COMPACT_LOOK; ++k)
              if ((st[k] >> 32) != tag) st[k] = hi | CST_TOTAL;
            break;
          }
#pragma unroll
          for (int k = 0; k < COMPACT_LOOK; ++k) {
            const int64_t q = j - 64 * k - lane;
            if ((st[k] >> 32) != tag) st[k] = cst_load(&w.cstat[q]);
          }
        }
        bool done = false;
#pragma unroll
        for (int k = 0; k < COMPACT_LOOK; ++k) {
          if (done) break;  // wave-uniform
          const uint64_t tm = __ballot(((uint32_t)st[k] & CST_TOTAL) != 0);
          const int l = tm ? __builtin_ctzll(tm) : 64;
          const uint32_t val = lane <= l ? ((uint32_t)st[k] & ~CST_TOTAL) : 0u;
          base += (uint32_t)__builtin_amdgcn_readlane((int)wave_incl_scan(val, lane), 63);
          done = tm != 0;
        }
        if (done) break;
      }
      if (lane == 0) cst_store(&w.cstat[b], hi | CST_TOTAL | (base + tot));
    }
    if (lane == 0) {
      sbase = base;
      w.blkprefix[b] = base;
      if (!ok) atomicOr(w.status, ST_STALL);
    }
  }
  __syncthreads();
  // contiguous stores of the staged ids (id j of the block is wave g's
  // j - pre[g]-th, g the last wave with pre[g] <= j)
  const uint32_t base = sbase;
  for (uint32_t j = tid; j < tot; j += COMPACT_TPB) {
    int g = 0;
#pragma unroll
    for (int q = 1; q < COMPACT_TPB / 64; ++q) g += j >= pre[q];
    if (base + j < w.out_cap) w.out[base + j] = sout[g * CW + (j - pre[g])];
  }
  if (b == nblk - 1 && tid == 0) {
    const uint32_t total = base + tot;
    w.blkprefix[nblk] = total;
    w.status[1] = total;
    if (total > w.out_cap) atomicOr(w.status, ST_CAPACITY);
    if (w.gate) {
      // every earlier stage that sets status bits or failed cuts has ended
      w.gate[GATE_STATUS] = atomicOr(w.status, 0u);
      w.gate[GATE_TOTAL] = total;
      w.gate[GATE_FAIL] = *w.nfail;
      w.gate[GATE_NLIT] = w.nlit ? *w.nlit : 0u;
      w.gate[GATE_PASS] = w.npass ? *w.npass : 0u;
      __threadfence_system();
      w.gate[GATE_DONE] = w.seq;
      __threadfence_system();
    }
  }
}

hipError_t launch_compact(const DevWork& w, hipStream_t s, uint32_t tag,
                          hipEvent_t start, hipEvent_t stop) {
  const int64_t nblk = (w.nb + COMPACT_BLOCK - 1) / COMPACT_BLOCK;
  launch_ev(k_compact, dim3((uint32_t)(nblk > 0 ? nblk : 1)), dim3(COMPACT_TPB), s,
            start, stop, w, nblk > 0 ? nblk : 1, tag);
  return hipGetLastError();
}

// ------------------------------------------------- session-seed checkpoints
// The session store adopts an encoding as ids plus sparse span checkpoints:
// for token k * stride (k = 0, 1, ...) its first byte, the first byte of
// the character holding it, and that character's index
// (crates/toktier-store-core/src/tail.rs:17-31, :173-205). Token j's id
// sits at its first byte in tok, and k_compact leaves the tokens before
// each COMPACT_BLOCK-byte block in blkprefix, so a checkpoint is found in
// one block.

// characters (UTF-8 lead bytes) of each COMPACT_BLOCK-byte block
__global__ __launch_bounds__(COMPACT_TPB) void k_seed_chars(const uint8_t* text,
                                                            int64_t nb,
                                                            uint32_t* ccount) {
  const int64_t p0 = (int64_t)blockIdx.x * COMPACT_BLOCK +
                     (int64_t)threadIdx.x * COMPACT_PER_THREAD;
  uint32_t c = 0;
  for (int k = 0; k < COMPACT_PER_THREAD; ++k) {
    const int64_t p = p0 + k;
    if (p < nb) c += !is_cont(text[p]);
  }
  uint32_t tot;
  block_excl_scan(c, &tot);
  if (threadIdx.x == 0) ccount[blockIdx.x] = tot;
}

// exclusive scan of the block counts, in place (one workgroup)
__global__ __launch_bounds__(COMPACT_TPB) void k_seed_scan(uint32_t* ccount,
                                                           int64_t nblk) {
  uint32_t carry = 0;
  for (int64_t base = 0; base < nblk; base += COMPACT_TPB) {
    const int64_t j = base + threadIdx.x;
    const uint32_t v = j < nblk ? ccount[j] : 0u;
    uint32_t tot;
    const uint32_t ex = block_excl_scan(v, &tot);
    if (j < nblk) ccount[j] = carry + ex;
    carry += tot;
  }
}

// one workgroup per checkpoint k = first + blockIdx.x: token T = k * stride
// (T < the token count, which the host checks); pts[3k..3k+2] = byte,
// anchor byte, anchor character
__global__ __launch_bounds__(COMPACT_TPB) void k_seed_points(
    const uint32_t* tok, const uint8_t* text, int64_t nb,
    const uint32_t* blkprefix, int64_t nblk, const uint32_t* cprefix,
    uint32_t stride, uint32_t first, uint64_t* pts) {
  __shared__ unsigned long long s_lo;
  __shared__ int64_t s_pos;
  const int tid = threadIdx.x;
  const int64_t kpt = (int64_t)first + blockIdx.x;
  const uint64_t T = (uint64_t)kpt * stride;
  // The block holding token T: the last b in [0, nblk) with blkprefix[b]
  // <= T (non-decreasing, blkprefix[0] = 0). Each round the workgroup
  // samples COMPACT_TPB evenly spaced candidates of [lo, hi) and keeps the
  // span after the last one at or below T: two rounds for a 4 MiB request.
  int64_t lo = 0, hi = nblk;
  while (hi - lo > 1) {
    const int64_t step = (hi - lo + COMPACT_TPB - 1) / COMPACT_TPB;
    if (tid == 0) s_lo = (unsigned long long)lo;
    __syncthreads();
    const int64_t j = lo + (int64_t)tid * step;
    if (j < hi && blkprefix[j] <= T) atomicMax(&s_lo, (unsigned long long)j);
    __syncthreads();
    lo = (int64_t)s_lo;
    hi = lo + step < hi ? lo + step : hi;
    __syncthreads();  // every thread has read s_lo before the next round
  }
  if (tid == 0) s_pos = -1;
  __syncthreads();
  const int64_t b = lo;
  const uint64_t r = T - blkprefix[b];
  const int64_t p0 = b * COMPACT_BLOCK + (int64_t)tid * COMPACT_PER_THREAD;
  uint32_t c = 0;
  for (int k = 0; k < COMPACT_PER_THREAD; ++k) {
    const int64_t p = p0 + k;
    c += p < nb && tok[p] != INVALID_ID;
  }
  uint32_t tot;
  const uint32_t ex = block_excl_scan(c, &tot);
  if (r >= ex && r < (uint64_t)ex + c) {
    uint64_t q = ex;
    for (int k = 0; k < COMPACT_PER_THREAD; ++k) {
      const int64_t p = p0 + k;
      if (p < nb && tok[p] != INVALID_ID) {
        if (q == r) { s_pos = p; break; }
        ++q;
      }
    }
  }
  __syncthreads();
  const int64_t pos = s_pos;
  if (pos < 0) {  // not reached when T is below the token count
    if (tid == 0) pts[3 * kpt] = ~0ULL;
    return;
  }
  int64_t a = pos;
  while (a > 0 && is_cont(text[a])) --a;
  // characters before a: the blocks before a's, then a's block up to a
  const int64_t ab = a / COMPACT_BLOCK;
  const int64_t q0 = ab * COMPACT_BLOCK + (int64_t)tid * COMPACT_PER_THREAD;
  uint32_t lc = 0;
  for (int k = 0; k < COMPACT_PER_THREAD; ++k) {
    const int64_t p = q0 + k;
    if (p < a) lc += !is_cont(text[p]);
  }
  uint32_t ltot;
  block_excl_scan(lc, &ltot);
  if (tid == 0) {
    uint64_t* o = pts + 3 * kpt;
    o[0] = (uint64_t)pos;
    o[1] = (uint64_t)a;
    o[2] = (uint64_t)cprefix[ab] + ltot;
  }
}

hipError_t launch_seed(const DevWork& w, const uint8_t* text, int64_t nb,
                       uint32_t n_points, uint32_t stride, uint32_t* ccount,
                       uint64_t* pts, hipStream_t s) {
  const int64_t nblk = (nb + COMPACT_BLOCK - 1) / COMPACT_BLOCK;
  if (nblk <= 0 || n_points == 0) return hipSuccess;
  hipLaunchKernelGGL(k_seed_chars, dim3((uint32_t)nblk), dim3(COMPACT_TPB), 0,
                     s, text, nb, ccount);
  hipLaunchKernelGGL(k_seed_scan, dim3(1), dim3(COMPACT_TPB), 0, s, ccount, nblk);
  // launches of at most 2^22 workgroups (grid size times workgroup size
  // stays below 2^32)
  constexpr uint32_t CHUNK = 1u << 22;
  for (uint32_t first = 0; first < n_points; first += CHUNK) {
    const uint32_t n = n_points - first < CHUNK ? n_points - first : CHUNK;
    hipLaunchKernelGGL(k_seed_points, dim3(n), dim3(COMPACT_TPB), 0, s,
                       (const uint32_t*)w.tok, text, nb,
                       (const uint32_t*)w.blkprefix, nblk,
                       (const uint32_t*)ccount, stride, first, pts);
  }
  return hipGetLastError();
}

// row d starts at the number of tokens whose first byte lies before
// doc_offsets[d]: the compaction's prefix at its block plus the token slots
// of the block before it, counted by one wave (lanes strided, then a wave
// sum)
__global__ __launch_bounds__(256) void k_doc_offsets(DevWork w,
                                                     const uint64_t* doc_offsets,
                                                     uint32_t n, uint64_t* rows) {
  const uint32_t d = blockIdx.x * 4 + wave_id();
  if (d > n) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  int64_t p = (int64_t)doc_offsets[d];
  if (p > w.nb) p = w.nb;
  const int64_t blk = p / COMPACT_BLOCK;
  uint32_t c = 0;
  for (int64_t q = blk * COMPACT_BLOCK + lane; q < p; q += 64)
    c += w.tok[q] != INVALID_ID;
  for (int o = 32; o > 0; o >>= 1) c += (uint32_t)__shfl_xor((int)c, o);
  if (lane == 0) rows[d] = (uint64_t)w.blkprefix[blk] + c;
}

// the document-start mask of a batch from its offsets: one thread per mask
// word, the documents that start in it found by a binary search
__global__ __launch_bounds__(256) void k_doc_mask(uint64_t* mask, int64_t nwords,
                                                  const uint64_t* offs,
                                                  uint32_t n_docs, int64_t nb) {
  const int64_t wd = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (wd >= nwords) return;
  const uint64_t lo = (uint64_t)wd * 64, hi = lo + 64;
  uint32_t a = 0, b = n_docs;  // first document with offs[d] >= lo
  while (a < b) {
    const uint32_t m = (a + b) / 2;
    if (offs[m] < lo) a = m + 1;
    else b = m;
  }
  uint64_t bits = 0;
  for (uint32_t d = a; d < n_docs && offs[d] < hi; ++d)
    if (offs[d] < (uint64_t)nb) bits |= 1ull << (offs[d] & 63);
  mask[wd] = bits;
}

hipError_t launch_doc_mask(uint64_t* mask, int64_t nwords,
                           const uint64_t* doc_offsets, uint32_t n_docs,
                           int64_t nb, hipStream_t s) {
  hipLaunchKernelGGL(k_doc_mask, dim3((uint32_t)((nwords + 255) / 256)),
                     dim3(256), 0, s, mask, nwords, doc_offsets, n_docs, nb);
  return hipGetLastError();
}

hipError_t launch_doc_offsets(const DevWork& w, const uint64_t* doc_offsets,
                              uint32_t n_docs, uint64_t* row_offsets,
                              hipStream_t s) {
  const uint32_t n = n_docs + 1;  // rows, one wave each
  hipLaunchKernelGGL(k_doc_offsets, dim3((n + 3) / 4), dim3(256), 0, s, w,
                     doc_offsets, n_docs, row_offsets);
  return hipGetLastError();
}

// ------------------------------------------- the allocation-free workspace

// The workspace of tk_engine_encode_device_noalloc: a file-scope device
// array, one copy per device. Host code reaches it only through the address
// scratch_region looks up.
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

hipError_t scratch_region(int device, uint8_t** p) {
  static std::mutex mu;
  static void* addr[64] = {};
  *p = nullptr;
  if (device < 0 || device >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(mu);
  if (!addr[device]) {
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != device && (e = hipSetDevice(device)) != hipSuccess) return e;
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != device) (void)hipSetDevice(cur);
    if (e != hipSuccess) return e;
    if (!ptr) return hipErrorInvalidSymbol;
    addr[device] = ptr;
  }
  *p = static_cast<uint8_t*>(addr[device]);
  return hipSuccess;
}

__global__ void k_clear(uint32_t* a, uint32_t na, uint64_t* b, uint32_t nb,
                        uint64_t* c, uint32_t nc) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < na) a[i] = 0;
  if (i < nb) b[i] = 0;
  if (i < nc) c[i] = 0;
}

hipError_t launch_clear(uint32_t* a, uint32_t na, uint64_t* b, uint32_t nb,
                        uint64_t* c, uint32_t nc, hipStream_t s) {
  uint32_t n = na > nb ? na : nb;
  n = n > nc ? n : nc;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_clear, dim3((n + 255) / 256), dim3(256), 0, s, a, na,
                     b, nb, c, nc);
  return hipGetLastError();
}

}  // namespace tk
