// tk_engine.cpp -- host side of the gfx950 fresh-encode engine and its
// C-ABI (include/toktier_hip.h).
//
// Mirrors the reference executor (crates/toktier-routing-core/src/gpu.rs):
// table validation (validate_tables :1642-1679), device open with an
// architecture check (Executor::new :248-344), a capacity-sized workspace
// reused across calls (ensure_workspace :370-381), one stream, the encode
// sequence H2D -> stages -> count read -> ids read (encode_in_workspace
// :570-600), and the batched channel with forced starts at document heads
// (Executor::encode_batch :605-750). Unlike the reference host, the NFC
// decision is taken on the device (quick check fused into the pretokenize
// stage); only a failing text goes back to the caller for exact
// normalization (TK_E_NEEDS_NFC).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "../../include/toktier_hip.h"
#include "tk_device.h"
#include "tk_staging.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HIP_TRY(call)                                                      \
  do {                                                                     \
    hipError_t e_ = (call);                                                \
    if (e_ != hipSuccess)                                                  \
      return fail(TK_E_DEVICE, "%s failed: %s (%s)", #call,                \
                  hipGetErrorName(e_), hipGetErrorString(e_));             \
  } while (0)

constexpr size_t PLANE = 0x110000;
// bound of a device wait on another workgroup's published word (ms)
constexpr int WAIT_MS = 100;

bool pow2(uint64_t x) { return x && !(x & (x - 1)); }

template <class T>
struct DevBuf {
  T* p = nullptr;
  size_t n = 0;
  ~DevBuf() { reset(); }
  void reset() {
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
  }
  hipError_t alloc(size_t count) {
    reset();
    void* q = nullptr;
    hipError_t e = hipMalloc(&q, count ? count * sizeof(T) : 1);
    if (e == hipSuccess) { p = static_cast<T*>(q); n = count; }
    return e;
  }
};

// 64-bit splitmix, the pair-table slot function (bpe_tables.py:107-111)
uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ULL;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
  return x ^ (x >> 31);
}

uint64_t host_pair_lookup(const uint64_t* keys, const uint64_t* vals,
                          uint64_t count, uint32_t l, uint32_t r) {
  const uint64_t key = ((uint64_t)l << 32) | r, mask = count - 1;
  uint64_t i = splitmix64(key) & mask;
  for (uint64_t probes = 0; probes < count; ++probes) {
    if (keys[i] == key) return vals[i];
    if (keys[i] == ~0ULL) return ~0ULL;
    i = (i + 1) & mask;
  }
  return ~0ULL;
}

// Compact pair table (tk_device.h): two candidate buckets of two slots per
// pair, filled by cuckoo placement (an entry that finds both buckets full
// displaces one of the residents to that resident's other bucket, and so
// on), at a load of at most 0.6; a table one size larger is tried when a
// placement walk runs too long. Returns false when the artifact does not fit
// the packing (ids >= 2^18, ranks >= 2^19 - 1); the engine then probes the
// interleaved boundary table instead.
using PairEntries = std::vector<std::pair<uint64_t, uint64_t>>;  // (key36, rank<<18|id)

// Cuckoo placement of the first n entries into 2^bits two-slot buckets
// (the compact table's layout); false when one does not fit.
bool place_pairs(const PairEntries& ent, size_t n, uint32_t bits,
                 std::vector<uint64_t>& out);

bool build_compact_pairs(const uint64_t* keys, const uint64_t* vals,
                         uint64_t count, std::vector<uint64_t>& out,
                         uint32_t& bits, PairEntries* entries) {
  PairEntries ent;
  for (uint64_t i = 0; i < count; ++i) {
    if (keys[i] == ~0ULL) continue;
    const uint64_t l = keys[i] >> 32, r = keys[i] & 0xFFFFFFFFULL;
    const uint64_t rank = vals[i] >> 32, id = vals[i] & 0xFFFFFFFFULL;
    if (l >= (1u << 18) || r >= (1u << 18) || id >= (1u << 18) ||
        rank >= (1u << 19) - 1)
      return false;
    ent.push_back({(l << 18) | r, (rank << 18) | id});
  }
  bits = tk::CTAB_MIN_BITS;
  while ((2ULL << bits) * 6 < ent.size() * 10) ++bits;
  for (; bits <= tk::CTAB_MAX_BITS; ++bits) {
    if (place_pairs(ent, ent.size(), bits, out)) {
      if (entries) *entries = std::move(ent);
      return true;
    }
  }
  return false;
}

// The hot-pair table: the rules of the lowest ranks, as many as the
// HOT_BITS buckets take; hot_k is one past the highest rank placed, so
// every rule of a rank below hot_k is in it (each rule has its own rank).
// False when not even the first rule fits.
bool build_hot_pairs(PairEntries ent, std::vector<uint64_t>& out, uint32_t& hot_k) {
  std::sort(ent.begin(), ent.end(),
            [](const auto& a, const auto& b) { return a.second < b.second; });
  size_t lo = 0, hi = std::min<size_t>(ent.size(), (size_t)2 << tk::HOT_BITS);
  while (lo < hi) {  // the largest count that fits
    const size_t mid = (lo + hi + 1) / 2;
    std::vector<uint64_t> t;
    if (place_pairs(ent, mid, tk::HOT_BITS, t)) lo = mid;
    else hi = mid - 1;
  }
  if (lo == 0 || !place_pairs(ent, lo, tk::HOT_BITS, out)) return false;
  hot_k = (uint32_t)(ent[lo - 1].second >> 18) + 1;
  return true;
}

bool place_pairs(const PairEntries& ent, size_t n, uint32_t bits,
                 std::vector<uint64_t>& out) {
  {
    const uint64_t nbk = 1ULL << bits;
    out.assign(nbk * 2, ~0ULL);
    uint64_t rng = 0x2545F4914F6CDD1DULL;
    bool ok = true;
    for (size_t ei = 0; ei < n; ++ei) {
      const auto& e = ent[ei];
      const uint64_t x = tk::pair_perm((uint32_t)(e.first >> 18),
                                       (uint32_t)(e.first & 0x3FFFF));
      // the entry being placed: tag, first bucket, rank<<18 | id, and the
      // bucket to try first
      uint32_t tag = (uint32_t)(x >> bits);
      uint32_t b1 = (uint32_t)(x & (nbk - 1));
      uint64_t low = e.second;
      uint32_t at = b1;
      bool placed = false;
      for (int kick = 0; kick < 512 && !placed; ++kick) {
        const uint32_t alt = tk::pair_alt(b1, tag, bits);
        const uint32_t other = at == b1 ? alt : b1;
        for (const uint32_t bk : {at, other}) {
          for (int k = 0; k < 2 && !placed; ++k) {
            uint64_t& slot = out[(uint64_t)bk * 2 + k];
            if (slot == ~0ULL) {
              slot = ((uint64_t)tag << 38) | ((uint64_t)(bk != b1) << 37) | low;
              placed = true;
            }
          }
          if (placed) break;
        }
        if (placed) break;
        // both full: take a resident's place in `at`; the resident moves on
        // to its other bucket (pair_alt is an involution for a fixed tag)
        rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17;
        uint64_t& victim = out[(uint64_t)at * 2 + (rng & 1)];
        const uint64_t v = victim;
        victim = ((uint64_t)tag << 38) | ((uint64_t)(at != b1) << 37) | low;
        tag = (uint32_t)(v >> 38);
        const bool vsecond = (v >> 37) & 1;
        b1 = vsecond ? tk::pair_alt(at, tag, bits) : at;
        low = v & ((1ULL << 37) - 1);
        at = vsecond ? b1 : tk::pair_alt(b1, tag, bits);
      }
      if (!placed) { ok = false; break; }
    }
    return ok;
  }
}

// One request's device workspace: every per-call buffer, carved out of one
// region -- the engine's own allocation, or, for
// tk_engine_encode_device_noalloc, the library's static scratch array.
// `slot` and `ctag` are the region's own call state: the control slot the
// next call uses (each call's k_pretok clears the other one) and the last
// compaction tag (the look-back status words carry it, so they are never
// cleared between calls).
struct Workspace {
  size_t cap = 0;  // input bytes the workspace holds
  uint8_t* text = nullptr;
  uint64_t *starts = nullptr, *docmask = nullptr, *heap = nullptr;
  uint64_t *cstat = nullptr, *inlong = nullptr, *cuts = nullptr;
  uint64_t *failm = nullptr, *hfirst = nullptr, *hlast = nullptr;
  uint64_t *dirty_cur = nullptr, *dirty_next = nullptr;
  uint64_t *lits = nullptr, *litb = nullptr, *docmask_lit = nullptr;
  uint64_t* nrun = nullptr;  // per k_pretok tile: the digit run, then two
                             // automaton words (o200k)
  uint32_t *tok = nullptr, *longlist = nullptr, *ctrl = nullptr;
  uint32_t *blkcount = nullptr, *blkprefix = nullptr;
  uint32_t *hmeta = nullptr, *seglist = nullptr, *plist = nullptr;
  uint32_t* wlist = nullptr;  // a repair pass's windows
  uint32_t* vlist = nullptr;  // the grid windows with long-piece bytes
  int32_t *nx = nullptr, *pv = nullptr;
  size_t long_pairs = 0, seg_pairs = 0, nblk = 0, tiles = 0;
  uint32_t slot = 0;
  uint32_t ctag = 0;
};

// Lays a workspace for `cap` input bytes out at `base` (each buffer
// 256-byte aligned) and returns the bytes it spans; base == nullptr only
// sizes it. About 70 bytes per input byte.
size_t carve(Workspace& w, uint8_t* base, size_t cap) {
  size_t at = 0;
  auto take = [&](auto*& p, size_t count) {
    using T = std::remove_reference_t<decltype(*p)>;
    at = (at + 255) & ~(size_t)255;
    p = base ? reinterpret_cast<T*>(base + at) : nullptr;
    at += (count ? count : 1) * sizeof(T);
  };
  const size_t words = cap / 64 + 8;
  const size_t nblk = cap / tk::COMPACT_BLOCK + 2;
  const size_t long_cap = cap / 32 + 64;
  const size_t seg_cap = cap / 2 + 64;
  const int64_t tiles = tk::pretok_tiles((int64_t)cap);
  take(w.text, cap + 64);
  take(w.starts, words);
  take(w.docmask, words);
  take(w.tok, cap + 64);
  take(w.nx, cap);
  take(w.pv, cap);
  take(w.heap, 3 * cap);
  take(w.longlist, 2 * long_cap);
  take(w.ctrl, 2 * tk::CTRL_WORDS);  // two control slots
  take(w.inlong, words);
  take(w.cuts, words);
  take(w.failm, words);
  take(w.hfirst, cap);
  take(w.hlast, cap);
  take(w.hmeta, cap);
  take(w.seglist, 2 * seg_cap);
  take(w.wlist, words);
  take(w.vlist, words);
  take(w.dirty_cur, words / 64 + 2);
  take(w.dirty_next, words / 64 + 2);
  take(w.blkcount, nblk);
  take(w.blkprefix, nblk);
  take(w.cstat, nblk);
  take(w.plist, (size_t)tk::PT_LOCAL_SLOTS * tiles);
  take(w.lits, words);
  take(w.litb, words);
  take(w.docmask_lit, words);
  take(w.nrun, 3 * (size_t)tiles);
  w.cap = cap;
  w.tiles = (size_t)tiles;
  w.long_pairs = long_cap;
  w.seg_pairs = seg_cap;
  w.nblk = nblk;
  return at;
}

}  // namespace

struct tk_engine {
  std::mutex mu;
  int device = 0;
  hipStream_t stream = nullptr;
  std::string family, sha, arch;
  tk_config cfg{};
  // tables
  DevBuf<uint8_t> cls, nfc, blob;
  DevBuf<ulonglong2> pairs, vocab;
  DevBuf<uint64_t> bytepair, ctab, hot;
  uint32_t hot_k = 0;  // rules of rank below it are in `hot`
  DevBuf<int32_t> byte_id;
  std::vector<uint8_t> host_nfc;
  tk::DevTables t{};
  // workspace (carved from one allocation) and the batch / seed buffers
  DevBuf<uint8_t> wsmem;
  Workspace ws;
  DevBuf<uint64_t> docoffs;
  // a batch's document offsets on their way in, and its row offsets, which
  // k_doc_offsets writes here over PCIe right after the compaction
  tk::PinnedBuf offs_pin, rows_pin;
  DevBuf<uint32_t> seedc;  // per-block character counts (session seed)
  DevBuf<uint64_t> seedp;  // span checkpoints of the host-buffer seed
  // test-only: a host-buffer call whose input holds these bytes fails as a
  // whole after its pipeline ran (tk_engine_set_fault_marker)
  std::string fault_marker;
  DevBuf<uint32_t> unsafe;
  // added-token literals (tk_engine_set_added)
  DevBuf<uint64_t> lit_tab;
  DevBuf<uint8_t> lit_len;
  DevBuf<uint32_t> lit_id;
  tk::DevAdded added{};
  uint64_t last_literals = 0;
  size_t docs_cap = 0;
  // the static scratch array on this engine's device
  // (tk_engine_encode_device_noalloc)
  uint8_t* scratch = nullptr;
  uint32_t* host_ctrl = nullptr;  // pinned read-back of 8 control words
  // gate words: host memory the device writes mid-pipeline
  volatile uint32_t* gate = nullptr;
  uint32_t* gate_dev = nullptr;
  uint32_t seq = 0;
  // bound of a device wait on another workgroup (DevWork::wait_ticks):
  // WAIT_MS in ticks of the device's real-time counter
  uint64_t wait_ticks = 0;
  // TK_OPT_REPAIR_WIDEN: the first repair pass that widens the failed cuts
  // (k_fail_widen); 0: every piece over WIDE_MAX bytes merged whole, no
  // cuts (the path of tables that drop bytes)
  int repair_widen = tk::REPAIR_WIDEN;
  // timing
  int timing = 0;  // 0 off, 1 every kernel, 2 one kernel (timed_kernel)
  int timed_kernel = TK_KERNEL_BPE_PACK;
  hipEvent_t ev[8] = {};
  hipEvent_t kev[TK_KERNELS][2] = {};  // mode 1: each kernel's own dispatch
  double last_kus[TK_KERNELS] = {};
  // side stream for the long-piece stages, and its fork / join events
  hipStream_t stream2 = nullptr;
  hipEvent_t ev_join = nullptr;  // side stream -> engine stream
  // pieces over WIDE_MAX bytes (cut / segment / certify) on a stream of
  // their own, beside the 129..WIDE_MAX-byte merges of stream2
  hipStream_t stream3 = nullptr;
  hipEvent_t ev_join3 = nullptr;
  // host-to-host entries: pinned staging of the request bytes and of the
  // ids (written there by the compaction kernel), and the copy threads
  tk::PinnedBuf pin_in, pin_out;
  std::unique_ptr<tk::CopyPool> pool;
  double last_us[8] = {};
  size_t last_passes = 0;
  uint32_t last_nlong = 0, last_big = 0;
};

namespace {

int validate(const tk_config* cfg, const uint8_t* class_table, size_t class_len, size_t pk_len,
             size_t pv_len, size_t byte_id_len, size_t vk_len, size_t vv_len,
             size_t unsafe_len) {
  if (!cfg) return fail(TK_E_INVALID_ARG, "config is null");
  if (cfg->abi_version != TK_ABI_VERSION)
    return fail(TK_E_INVALID_ARG, "abi_version %u != %u", cfg->abi_version,
                TK_ABI_VERSION);
  if (cfg->ruleset != TK_RULESET_CL100K && cfg->ruleset != TK_RULESET_R50K &&
      cfg->ruleset != TK_RULESET_LAGUNA && cfg->ruleset != TK_RULESET_DEEPSEEK &&
      cfg->ruleset != TK_RULESET_O200K && cfg->ruleset != TK_RULESET_KIMI)
    return fail(TK_E_INVALID_ARG, "unsupported ruleset %d", cfg->ruleset);
  if (cfg->ruleset != TK_RULESET_R50K &&
      (cfg->digits_max < 1 || cfg->digits_max > 64))
    return fail(TK_E_INVALID_ARG, "digits_max %d out of range", cfg->digits_max);
  // the deepseek pattern has no contraction alternative; o200k rows come
  // with and without one; the others always have it
  if (cfg->ruleset != TK_RULESET_O200K &&
      (cfg->contractions != 0) != (cfg->ruleset != TK_RULESET_DEEPSEEK))
    return fail(TK_E_INVALID_ARG, "contractions=%d does not match ruleset %d",
                cfg->contractions, cfg->ruleset);
  // the kimi digit alternative is \p{N}{1,3}, counted in the split's state
  if (cfg->ruleset == TK_RULESET_KIMI && cfg->digits_max != 3)
    return fail(TK_E_INVALID_ARG, "digits_max %d: the kimi split groups digits by 3",
                cfg->digits_max);
  // shape rules of the reference executor (gpu.rs:1642-1679)
  if (class_len < PLANE)
    return fail(TK_E_SHAPE, "class table does not cover U+10FFFF");
  {
    // four classes (P L N S), seven for deepseek (O L M N PS WS CRLF) and
    // for o200k (P U L C N S M), ten for kimi (those and HL HN HP)
    const uint8_t top = cfg->ruleset == TK_RULESET_KIMI ? 9
                      : cfg->ruleset == TK_RULESET_DEEPSEEK ||
                        cfg->ruleset == TK_RULESET_O200K ? 6 : 3;
    uint8_t mx = 0;
    for (size_t i = 0; i < PLANE; ++i) mx = class_table[i] > mx ? class_table[i] : mx;
    if (mx > top)
      return fail(TK_E_SHAPE, "class table value %u above %u for ruleset %d",
                  mx, top, cfg->ruleset);
  }
  if (!pow2(cfg->pair_count) || pk_len != 8 * cfg->pair_count || pv_len != pk_len)
    return fail(TK_E_SHAPE, "pair tables have an invalid shape");
  if (!pow2(cfg->vocab_count) || vk_len != 8 * cfg->vocab_count || vv_len != vk_len)
    return fail(TK_E_SHAPE, "vocabulary tables have an invalid shape");
  if (byte_id_len != 256 * 4 || unsafe_len % 4 != 0)
    return fail(TK_E_SHAPE, "byte-id or unsafe-rank table has an invalid shape");
  return TK_OK;
}

int ensure_workspace(tk_engine* e, size_t nb, size_t n_docs) {
  size_t need = 1u << 16;
  while (need < nb) need <<= 1;
  if (need > (size_t)1 << 30) return fail(TK_E_CAPACITY, "input of %zu bytes exceeds 1 GiB", nb);
  if (need > e->ws.cap) {
    Workspace w;
    const size_t bytes = carve(w, nullptr, need);
    e->ws = Workspace{};
    HIP_TRY(e->wsmem.alloc(bytes));
    carve(e->ws, e->wsmem.p, need);
    // the control slots start clear, and the compaction status words carry
    // tags from 1 up, so zeroed words never match
    HIP_TRY(hipMemset(e->ws.ctrl, 0, 2 * tk::CTRL_WORDS * sizeof(uint32_t)));
    HIP_TRY(hipMemset(e->ws.cstat, 0, e->ws.nblk * sizeof(uint64_t)));
    HIP_TRY(hipMemset(e->ws.nrun, 0, 3 * e->ws.tiles * sizeof(uint64_t)));
  }
  if (n_docs + 1 > e->docs_cap) {
    HIP_TRY(e->docoffs.alloc(n_docs + 1));
    HIP_TRY(e->offs_pin.ensure((n_docs + 1) * sizeof(uint64_t)));
    HIP_TRY(e->rows_pin.ensure((n_docs + 1) * sizeof(uint64_t)));
    e->docs_cap = n_docs + 1;
  }
  return TK_OK;
}

tk::DevWork make_work(tk_engine* e, Workspace& ws, const uint8_t* d_text,
                      size_t nb, const uint64_t* d_docmask, bool check_nfc,
                      uint32_t* out, size_t out_cap, bool literals) {
  uint32_t* ctrl = ws.ctrl + ws.slot * tk::CTRL_WORDS;
  tk::DevWork w{};
  w.text = d_text;
  w.nb = (int64_t)nb;
  w.docmask = d_docmask;
  w.check_nfc = check_nfc ? 1 : 0;
  w.starts = ws.starts;
  w.tok = ws.tok;
  w.nx = ws.nx;
  w.pv = ws.pv;
  w.heap = ws.heap;
  w.longlist = ws.longlist;
  w.longcount = ctrl + tk::CTRL_LONG;
  w.long_cap = (uint32_t)ws.long_pairs;
  w.status = ctrl + tk::CTRL_STATUS;
  w.blkcount = ws.blkcount;
  w.blkprefix = ws.blkprefix;
  w.cstat = ws.cstat;
  w.out = out;
  w.out_cap = (uint32_t)std::min<size_t>(out_cap, 0xFFFFFFFFu);
  w.inlong = ws.inlong;
  w.cuts = ws.cuts;
  w.failm = ws.failm;
  w.hfirst = ws.hfirst;
  w.hlast = ws.hlast;
  w.hmeta = ws.hmeta;
  w.seglist = ws.seglist;
  w.segcount = ctrl + tk::CTRL_SEG;
  w.seg_cap = (uint32_t)ws.seg_pairs;
  w.wlist = ws.wlist;
  w.wcount = ctrl + tk::CTRL_WIN;
  w.wlist_cap = (uint32_t)(ws.cap / 64 + 8);
  w.nfail = ctrl + tk::CTRL_FAIL;
  w.nfail_prev = nullptr;
  w.npass = ctrl + tk::CTRL_PASS;
  w.dirty_cur = ws.dirty_cur;
  w.dirty_next = ws.dirty_next;
  w.plist = ws.plist;  // (tiles * PT_LOCAL_SLOTS < 2^32 for nb <= 1 GiB)
  w.pseg = ctrl + tk::CTRL_PSEG;
  w.nbig = ctrl + tk::CTRL_BIG;
  w.prepdone = ctrl + tk::CTRL_PREP;
  w.nwide = ctrl + tk::CTRL_WIDE;
  w.nrows = ctrl + tk::CTRL_ROWS;
  w.rowq = ctrl + tk::CTRL_ROWQ;
  w.vlist = ws.vlist;
  w.vcount = ctrl + tk::CTRL_VLIST;
  w.gate = e->gate_dev;
  w.seq = e->seq;
  w.wait_ticks = e->wait_ticks;
  w.ctrl_next = ws.ctrl + (ws.slot ^ 1) * tk::CTRL_WORDS;
  w.nlit = ctrl + tk::CTRL_NLIT;
  w.nrun = ws.nrun;
  w.ostate = ws.nrun + ws.tiles;
  w.lits = literals ? ws.lits : nullptr;
  w.litb = literals ? ws.litb : nullptr;
  w.clear_words = (int64_t)(nb / 64 + 4);
  w.clear_dwords = w.clear_words / 64 + 2;
  return w;
}

// Certification passes over the long pieces: pass 0 certifies every cut;
// repair pass p >= 1 drops the cuts pass p - 1 failed, redoes the joined
// segments and certifies them again, and runs only when pass p - 1 failed
// any cut (its count: the other of two alternating control words). Up to
// DEV_REPAIRS repair passes are queued on the long-piece stream without
// the host; the host continues only if cuts still fail after them.
constexpr int DEV_REPAIRS = 3;
uint32_t* fail_count(uint32_t* ctrl, int p) {
  return ctrl + ((p & 1) ? tk::CTRL_FAIL2 : tk::CTRL_FAIL);
}
tk::DevWork pass_work(const tk::DevWork& w, uint32_t* ctrl, int p) {
  tk::DevWork q = w;
  q.nfail = fail_count(ctrl, p);
  q.nfail_prev = p == 0 ? nullptr : fail_count(ctrl, p - 1);
  return q;
}

// The internal failures a call's status word can carry, each naming the
// stage that reported it (TK_OK when there is none).
int internal_status(uint32_t st) {
  if (st & tk::ST_LONGOVF) return fail(TK_E_INTERNAL, "piece queue overflow");
  if (st & tk::ST_STALL_PRETOK)
    return fail(TK_E_INTERNAL,
                "pretokenize look-back timed out (a tile's digit-run count or "
                "automaton state was not published within %d ms)", WAIT_MS);
  if (st & tk::ST_STALL)
    return fail(TK_E_INTERNAL,
                "compaction look-back timed out (a block's running total was "
                "not published within %d ms)", WAIT_MS);
  if (st & tk::ST_ROUNDS)
    return fail(TK_E_INTERNAL, "workgroup merge ran past its round bound");
  return TK_OK;
}

int read_ctrl_words(const uint32_t* ctrl, hipStream_t s, uint32_t* h) {
  HIP_TRY(hipMemcpyAsync(h, ctrl, 16 * sizeof(uint32_t),
                         hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  if (int rc = internal_status(h[tk::CTRL_STATUS])) return rc;
  return TK_OK;
}

// Wait until k_bpe_pack of call `seq` has written the gate words (a
// spin on host memory). A device fault would stop the writer, so after a
// generous bound the stream is synchronized to surface its error.
int wait_gate(tk_engine* e, uint32_t seq, hipStream_t s) {
  const auto t0 = std::chrono::steady_clock::now();
  for (uint64_t spin = 0;; ++spin) {
    if (e->gate[tk::GATE_SEQ] == seq) {
      std::atomic_thread_fence(std::memory_order_acquire);
      return TK_OK;
    }
    if ((spin & 1023) == 1023 &&
        std::chrono::steady_clock::now() - t0 > std::chrono::seconds(10)) {
      HIP_TRY(hipStreamSynchronize(s));
      if (e->gate[tk::GATE_SEQ] == seq) return TK_OK;
      return fail(TK_E_INTERNAL, "gate words were not written");
    }
  }
}

float elapsed_us(hipEvent_t a, hipEvent_t b) {
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, a, b) != hipSuccess) return 0.f;
  return ms * 1e3f;
}

// Runs every stage for nb bytes already at d_text and waits for the result:
// ids in out (when they fit out_cap; else ST_CAPACITY), status and total
// count returned. Long pieces whose cuts fail certification are redone here
// (host-driven passes, each removing the failed cuts) until every cut holds.
// Nothing is cleared from the host: k_pretok clears the per-call masks and
// the control slot of the next call, so the stages run back to back.
// Added-token literals (literals == true): k_added splits the request
// first; the split marks document starts, so k_pretok runs its
// document-mask instance, on a mask k_added writes whole (ws.docmask_lit:
// the caller's document starts, if any, are read from d_docmask and kept).
// A batch's row offsets, counted right after the compaction, before the
// call's one stream sync (offs: the document offsets on the device; rows:
// n + 1 entries, e.g. host-mapped).
struct RowsOut {
  const uint64_t* offs;
  uint32_t n;
  uint64_t* rows;
};

int run_pipeline(tk_engine* e, Workspace& ws, const uint8_t* d_text,
                 size_t nb, const uint64_t* d_docmask, bool check_nfc,
                 hipStream_t s, uint32_t* out, size_t out_cap,
                 uint32_t* status, uint32_t* total,
                 const tk::DevAdded* docs = nullptr,
                 const RowsOut* rows_out = nullptr) {
  ++e->seq;
  const bool literals = docs != nullptr;
  const uint64_t* host_dm = d_docmask;
  if (literals) d_docmask = ws.docmask_lit;
  const tk::DevWork w = make_work(e, ws, d_text, nb, d_docmask, check_nfc,
                                  out, out_cap, literals);
  uint32_t* ctrl = ws.ctrl + ws.slot * tk::CTRL_WORDS;
  hipEvent_t* ev = e->ev;
  // Timing mode 1: every kernel of TK_KERNEL_* takes a start / stop event
  // pair on its own dispatch (kev), and ev[3] marks the end of the side
  // streams' work (when they have any) on the engine stream; the stage
  // boundaries are read from those. Mode 2: ev[1] / ev[2] are the start /
  // end of the dispatch of the kernel TK_OPT_TIMED_KERNEL names only. (Each
  // timed dispatch delays the next one by a few microseconds, so the timed
  // loop of a benchmark uses mode 2.)
  const bool stages = e->timing == 1, one = e->timing == 2;
  auto ks = [&](int k) -> hipEvent_t {
    return stages ? e->kev[k][0] : one && e->timed_kernel == k ? ev[1] : nullptr;
  };
  auto ke = [&](int k) -> hipEvent_t {
    return stages ? e->kev[k][1] : one && e->timed_kernel == k ? ev[2] : nullptr;
  };
  bool launched[TK_KERNELS] = {};
  if (literals) {
    HIP_TRY(tk::launch_added(*docs, w, host_dm, s, ks(TK_KERNEL_ADDED),
                             ke(TK_KERNEL_ADDED)));
    launched[TK_KERNEL_ADDED] = true;
  }
  HIP_TRY(tk::launch_pretok(e->t, w, s, ks(TK_KERNEL_PRETOK), ke(TK_KERNEL_PRETOK)));
  launched[TK_KERNEL_PRETOK] = true;
  hipStream_t s2 = e->stream2, s3 = e->stream3;
  ws.slot ^= 1;  // this call's k_pretok clears the other slot
  // (k_bpe_pack's first waves resolve the long pieces' ends and open the
  // gate before they take their work units; its first units are the long
  // pieces of up to 128 bytes)
  HIP_TRY(tk::launch_bpe_pack(e->t, w, s, ks(TK_KERNEL_BPE_PACK),
                              ke(TK_KERNEL_BPE_PACK)));
  launched[TK_KERNEL_BPE_PACK] = true;
  // The gate words tell, while the packed merge runs, how many pieces are
  // over 64 bytes, how many of them have 129..256 bytes, 257..WIDE_MAX bytes
  // and more. Only then do the stages of those pieces go on the side streams,
  // beside k_bpe_pack, and only those with work: they need the long
  // pieces' ends alone, which the device had written and made visible
  // before it opened the gate, so no event orders them.
  int grc = wait_gate(e, w.seq, s);
  if (grc != TK_OK) return grc;
  const uint32_t nlong = e->gate[tk::GATE_NLONG];
  const uint32_t nrows = e->gate[tk::GATE_NROWS];
  const uint32_t nwide = e->gate[tk::GATE_NWIDE];
  // (cut / segment / certify, unless the pieces over WIDE_MAX bytes are
  // merged whole: tables that drop bytes, or TK_OPT_REPAIR_WIDEN 0)
  const bool cut = e->t.cert && e->repair_widen > 0;
  const uint32_t big = cut ? e->gate[tk::GATE_BIG] : 0;
  e->last_nlong = nlong;
  e->last_big = e->gate[tk::GATE_BIG];
  // (pieces of 65..128 bytes are k_bpe_rows' too past PACK_ROWS_MAX)
  const bool rows = nrows > 0 || nlong > (uint32_t)tk::PACK_ROWS_MAX;
  const bool side2 = rows || nwide > 0 ||
                     (!cut && e->gate[tk::GATE_BIG] > 0);
  {
    // two independent jobs on two side streams: the cut / segment / certify
    // path of the pieces over WIDE_MAX bytes (the request's critical path
    // when there are any), and the pieces of 129..WIDE_MAX bytes merged
    // whole (they touch disjoint bytes and read the same lists)
    if (big) {
      // cut / segment / certify, then the repair passes, all on their own
      // stream beside the packed merge and the wide merges
      HIP_TRY(tk::launch_long_windows(e->t, w, s3, ks(TK_KERNEL_LONG_WINDOWS),
                                      ke(TK_KERNEL_LONG_WINDOWS)));
      launched[TK_KERNEL_LONG_WINDOWS] = true;
      // the row merges next (their launch is not held behind the chain's
      // twenty-odd launches on the host)
      if (rows) {
        HIP_TRY(tk::launch_bpe_rows(e->t, w, s2, nlong, ks(TK_KERNEL_BPE_ROWS),
                                    ke(TK_KERNEL_BPE_ROWS)));
        launched[TK_KERNEL_BPE_ROWS] = true;
      }
      HIP_TRY(tk::launch_long_segments(e->t, w, s3));
      HIP_TRY(tk::launch_seg_lists(e->t, w, s3));
      HIP_TRY(tk::launch_certify(e->t, w, 1, s3));
      for (int p = 1; p <= DEV_REPAIRS; ++p) {
        const tk::DevWork wp = pass_work(w, ctrl, p);
        HIP_TRY(tk::launch_apply_fail(wp, s3, tk::repair_width(p, e->repair_widen)));
        HIP_TRY(tk::launch_repair_segments(e->t, wp, s3));
        HIP_TRY(tk::launch_certify(e->t, wp, 0, s3));
      }
      HIP_TRY(hipEventRecord(e->ev_join3, s3));
      HIP_TRY(hipStreamWaitEvent(s, e->ev_join3, 0));
    }
    // (after the chain's first kernel, so that one is dispatched first)
    if (rows && !big) {
      HIP_TRY(tk::launch_bpe_rows(e->t, w, s2, nlong, ks(TK_KERNEL_BPE_ROWS),
                                  ke(TK_KERNEL_BPE_ROWS)));
      launched[TK_KERNEL_BPE_ROWS] = true;
    }
    if (nwide > 0) HIP_TRY(tk::launch_bpe_wide(e->t, w, s2, nullptr, nlong));
    // (a table that drops bytes merges its pieces over WIDE_MAX bytes
    // whole, a workgroup each, after the wide merges)
    if (!cut && e->gate[tk::GATE_BIG] > 0)
      HIP_TRY(tk::launch_long_block(e->t, w, s2));
  }
  if (side2) {
    HIP_TRY(hipEventRecord(e->ev_join, s2));
    HIP_TRY(hipStreamWaitEvent(s, e->ev_join, 0));
  }
  // (the end of the side streams, or of the packed merge if later)
  const bool side = side2 || big;
  if (stages && side) HIP_TRY(hipEventRecord(ev[3], s));
  // the compaction reports the failed cuts left after the last queued pass
  tk::DevWork wc = w;
  if (big) wc.nfail = fail_count(ctrl, DEV_REPAIRS);
  HIP_TRY(tk::launch_compact(wc, s, ++ws.ctag, ks(TK_KERNEL_COMPACT),
                             ke(TK_KERNEL_COMPACT)));
  launched[TK_KERNEL_COMPACT] = true;
  if (rows_out)
    HIP_TRY(tk::launch_doc_offsets(w, rows_out->offs, rows_out->n, rows_out->rows, s));
  // k_compact's last block has left the outcome in the gate words: no
  // read-back copy
  HIP_TRY(hipStreamSynchronize(s));
  uint32_t* h = e->host_ctrl;
  if (e->gate[tk::GATE_DONE] != w.seq)
    return fail(TK_E_INTERNAL, "outcome words were not written");
  h[tk::CTRL_STATUS] = e->gate[tk::GATE_STATUS];
  h[tk::CTRL_TOTAL] = e->gate[tk::GATE_TOTAL];
  uint32_t residual = e->gate[tk::GATE_FAIL];
  e->last_passes = e->gate[tk::GATE_PASS];
  e->last_literals = literals && docs->n ? e->gate[tk::GATE_NLIT] : 0;
  if (int rc = internal_status(h[tk::CTRL_STATUS])) return rc;
  int rc = TK_OK;
  if (stages) {
    // [2]: how far the long-piece stages ran past the packed merge
    hipEvent_t t0ev = e->kev[literals ? TK_KERNEL_ADDED : TK_KERNEL_PRETOK][0];
    const double t1 = elapsed_us(t0ev, e->kev[TK_KERNEL_PRETOK][1]);
    const double t2 = elapsed_us(t0ev, e->kev[TK_KERNEL_BPE_PACK][1]);
    const double t3 = side ? elapsed_us(t0ev, ev[3]) : 0.0;
    const double t4 = elapsed_us(t0ev, e->kev[TK_KERNEL_COMPACT][1]);
    e->last_us[0] = t1;
    e->last_us[1] = t2 - t1;
    e->last_us[2] = t3 > t2 ? t3 - t2 : 0.0;
    e->last_us[3] = t4 - (t3 > t2 ? t3 : t2);
    e->last_us[4] = t4;
    for (int k = 0; k < TK_KERNELS; ++k)
      e->last_kus[k] = launched[k] ? elapsed_us(e->kev[k][0], e->kev[k][1]) : 0.0;
  } else if (one) {
    for (double& x : e->last_us) x = 0.0;
    e->last_us[1] = launched[e->timed_kernel] ? elapsed_us(ev[1], ev[2]) : 0.0;
  }
  if (residual != 0) {
    // cuts still fail after the queued passes: more passes from the host,
    // one at a time. From pass REPAIR_WIDEN on each failed cut also drops
    // 4^(p - REPAIR_WIDEN + 1) cuts on each side, so a cascade of L cuts
    // ends within about log4(L) passes; the bound (a width past 2^30 cuts)
    // only guards against a defect.
    int p = DEV_REPAIRS;
    if (stages) HIP_TRY(hipEventRecord(ev[5], s));
    while (residual != 0) {
      if (++p > std::max(DEV_REPAIRS, e->repair_widen) + 16)
        return fail(TK_E_INTERNAL, "certification did not converge");
      const tk::DevWork wp = pass_work(w, ctrl, p);
      HIP_TRY(tk::launch_apply_fail(wp, s, tk::repair_width(p, e->repair_widen)));
      HIP_TRY(tk::launch_repair_segments(e->t, wp, s));
      HIP_TRY(tk::launch_certify(e->t, wp, 0, s));
      if ((rc = read_ctrl_words(ctrl, s, h)) != TK_OK) return rc;
      residual = h[(p & 1) ? tk::CTRL_FAIL2 : tk::CTRL_FAIL];
    }
    if (stages) HIP_TRY(hipEventRecord(ev[6], s));
    wc.nfail = fail_count(ctrl, p);
    HIP_TRY(tk::launch_compact(wc, s, ++ws.ctag));
    if (stages) HIP_TRY(hipEventRecord(ev[7], s));
    // (the row offsets again, over the final compaction)
    if (rows_out)
      HIP_TRY(tk::launch_doc_offsets(w, rows_out->offs, rows_out->n, rows_out->rows, s));
    if ((rc = read_ctrl_words(ctrl, s, h)) != TK_OK) return rc;
    if (stages) {
      e->last_us[2] += elapsed_us(ev[5], ev[6]);
      e->last_us[3] = elapsed_us(ev[6], ev[7]);
      e->last_us[4] = elapsed_us(e->kev[literals ? TK_KERNEL_ADDED : TK_KERNEL_PRETOK][0],
                                 ev[7]);
    }
    e->last_passes = h[tk::CTRL_PASS];
  }
  *status = h[tk::CTRL_STATUS];
  *total = h[tk::CTRL_TOTAL];
  return TK_OK;
}

// ---- host <-> device through the pinned staging
constexpr size_t STAGE_SMALL = (size_t)256 << 10;  // one copy, this thread
constexpr size_t STAGE_CHUNK = (size_t)64 << 10;   // one claim of the copy threads

tk::CopyPool* copy_pool(tk_engine* e) {
  if (!e->pool) e->pool.reset(new tk::CopyPool(tk::copy_threads()));
  return e->pool.get();
}

// Page-locked (pinned, device-visible) host memory, e.g. from
// hipHostMalloc: the device's address of p, or nullptr for pageable memory.
// A pageable pointer makes the query fail (hipErrorInvalidValue); that
// error is taken back at once so no later check reports it.
uint8_t* pinned_dev(const void* p) {
  hipPointerAttribute_t a{};
  if (hipPointerGetAttributes(&a, p) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (a.type != hipMemoryTypeHost || !a.devicePointer || !a.hostPointer) return nullptr;
  return static_cast<uint8_t*>(a.devicePointer) +
         (static_cast<const uint8_t*>(p) - static_cast<const uint8_t*>(a.hostPointer));
}

// the device's address of [p, p + bytes) when the whole range lies in one
// page-locked allocation, else nullptr. Both ends mapping at the right
// distance is not enough (two adjacent allocations can): the allocation
// that holds the first byte must also hold the last one. A failed range
// query takes the staged path.
uint8_t* pinned_range(const void* p, size_t bytes) {
  if (bytes == 0) return nullptr;
  uint8_t* d0 = pinned_dev(p);
  if (!d0) return nullptr;
  uint8_t* d1 = pinned_dev(static_cast<const uint8_t*>(p) + bytes - 1);
  if (!d1 || (size_t)(d1 - d0) != bytes - 1) return nullptr;
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, d0) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  const uint8_t* b = static_cast<const uint8_t*>(base);
  return d0 >= b && (size_t)(d0 - b) + bytes <= size ? d0 : nullptr;
}

// n bytes between host buffers by the copy threads and this thread
void host_copy(tk_engine* e, uint8_t* dst, const uint8_t* src, size_t n) {
  if (n <= STAGE_SMALL) {
    std::memcpy(dst, src, n);
    return;
  }
  copy_pool(e)->run((n + STAGE_CHUNK - 1) / STAGE_CHUNK, [&](size_t k) {
    const size_t off = k * STAGE_CHUNK;
    std::memcpy(dst + off, src + off, std::min(STAGE_CHUNK, n - off));
  });
}

// n request bytes at src (host) into d_dst (device) on stream s: page-locked
// bytes in one transfer; pageable ones copied into the pinned staging
// first, then one transfer (the staging is free again once the call has
// synchronized, as every host entry does before it returns).
int stage_in(tk_engine* e, uint8_t* d_dst, const uint8_t* src, size_t n,
             hipStream_t s) {
  if (pinned_range(src, n)) {
    HIP_TRY(hipMemcpyAsync(d_dst, src, n, hipMemcpyHostToDevice, s));
    return TK_OK;
  }
  HIP_TRY(e->pin_in.ensure(std::max(n, e->ws.cap) + 64));
  host_copy(e, e->pin_in.p, src, n);
  HIP_TRY(hipMemcpyAsync(d_dst, e->pin_in.p, n, hipMemcpyHostToDevice, s));
  return TK_OK;
}

// Where the compaction kernel writes a host call's ids: straight into the
// caller's buffer when it is page-locked and 4-byte aligned (capacity
// ids_cap), else into the pinned out staging (capacity ws.cap), which
// ids_from_staging copies to the caller afterwards.
struct HostOut {
  uint32_t* dev = nullptr;  // the device's address of the target
  size_t cap = 0;
  bool staged = false;
};
int host_out(tk_engine* e, uint32_t* ids, size_t ids_cap, HostOut* o) {
  if (ids_cap > 0 && ((uintptr_t)ids & 3) == 0) {
    if (uint8_t* d = pinned_range(ids, ids_cap * sizeof(uint32_t))) {
      *o = {reinterpret_cast<uint32_t*>(d), ids_cap, false};
      return TK_OK;
    }
  }
  HIP_TRY(e->pin_out.ensure(e->ws.cap * sizeof(uint32_t) + 64));
  *o = {reinterpret_cast<uint32_t*>(e->pin_out.dev), e->ws.cap, true};
  return TK_OK;
}
void ids_from_staging(tk_engine* e, const HostOut& o, uint32_t* ids, size_t n) {
  if (o.staged && n)
    host_copy(e, reinterpret_cast<uint8_t*>(ids), e->pin_out.p, n * sizeof(uint32_t));
}

// host-side checks used only on a batch whose device status flagged a
// failure, to find the failing rows
bool host_utf8_ok(const uint8_t* s, size_t n) {
  size_t i = 0;
  while (i < n) {
    uint32_t b0 = s[i], v;
    int need;
    if (b0 < 0x80) { ++i; continue; }
    if (b0 < 0xC0) return false;
    if (b0 < 0xE0) { need = 1; v = b0 & 0x1F; }
    else if (b0 < 0xF0) { need = 2; v = b0 & 0x0F; }
    else if (b0 < 0xF8) { need = 3; v = b0 & 7; }
    else return false;
    for (int k = 1; k <= need; ++k) {
      if (i + k >= n || (s[i + k] & 0xC0) != 0x80) return false;
      v = (v << 6) | (s[i + k] & 0x3F);
    }
    if ((need == 1 && v < 0x80) || (need == 2 && v < 0x800) ||
        (need == 3 && v < 0x10000) || v > 0x10FFFF || (v >= 0xD800 && v <= 0xDFFF))
      return false;
    i += need + 1;
  }
  return true;
}

bool host_nfc_ok(const std::vector<uint8_t>& qc, const uint8_t* s, size_t n) {
  size_t i = 0;
  uint8_t prev = 0;
  bool first = true;
  while (i < n) {
    uint32_t b0 = s[i], v;
    int need = b0 < 0x80 ? 0 : b0 < 0xE0 ? 1 : b0 < 0xF0 ? 2 : 3;
    v = need == 0 ? b0 : need == 1 ? (b0 & 0x1F) : need == 2 ? (b0 & 0x0F) : (b0 & 7);
    for (int k = 1; k <= need && i + k < n; ++k) v = (v << 6) | (s[i + k] & 0x3F);
    if (v >= PLANE) return false;
    const uint8_t q = qc[v];
    if (q == 255 || (!first && q != 0 && prev > q)) return false;
    prev = q;
    first = false;
    i += need + 1;
  }
  return true;
}

// The document-start pass (k_added) ahead of k_pretok: the literal split
// (unless the caller did it: TK_FLAG_NO_ADDED) and Laguna's newline-run
// parts. Null when the call needs neither.
const tk::DevAdded* doc_pass(tk_engine* e, uint32_t flags, tk::DevAdded* a) {
  *a = e->added;
  if (flags & TK_FLAG_NO_ADDED) a->n = 0;
  return (a->n > 0 || a->newline_cuts) ? a : nullptr;
}

bool utf8_ok(const uint8_t* s, size_t n) { return host_utf8_ok(s, n); }

// a proper suffix of x is a prefix of y, or one holds the other
bool can_overlap(const std::string& x, const std::string& y) {
  if (x.find(y) != std::string::npos || y.find(x) != std::string::npos)
    return true;
  for (size_t k = 1; k < x.size() && k < y.size() + 1; ++k)
    if (k <= y.size() && x.compare(x.size() - k, k, y, 0, k) == 0) return true;
  return false;
}

}  // namespace

extern "C" {

const char* tk_last_error(void) { return g_err.c_str(); }

int tk_engine_preflight(const tk_config* cfg, const uint8_t* class_table,
                        size_t class_len, const uint64_t* pair_keys,
                        size_t pair_keys_len, const uint64_t* pair_vals,
                        size_t pair_vals_len, const int32_t* byte_id,
                        size_t byte_id_len, const uint64_t* vocab_keys,
                        size_t vocab_keys_len, const uint64_t* vocab_vals,
                        size_t vocab_vals_len, const uint32_t* unsafe_bits,
                        size_t unsafe_len) {
  if (!class_table || !pair_keys || !pair_vals || !byte_id || !vocab_keys ||
      !vocab_vals)
    return fail(TK_E_INVALID_ARG, "a table pointer is null");
  (void)unsafe_bits;
  return validate(cfg, class_table, class_len, pair_keys_len, pair_vals_len, byte_id_len,
                  vocab_keys_len, vocab_vals_len, unsafe_len);
}

int tk_engine_open(const tk_config* cfg, const uint8_t* class_table,
                   size_t class_len, const uint64_t* pair_keys,
                   size_t pair_keys_len, const uint64_t* pair_vals,
                   size_t pair_vals_len, const int32_t* byte_id,
                   size_t byte_id_len, const uint64_t* vocab_keys,
                   size_t vocab_keys_len, const uint64_t* vocab_vals,
                   size_t vocab_vals_len, const uint8_t* vocab_blob,
                   size_t vocab_blob_len, const uint32_t* unsafe_bits,
                   size_t unsafe_len, const uint8_t* nfc_qc,
                   size_t nfc_qc_len, tk_engine** out) {
  if (!out) return fail(TK_E_INVALID_ARG, "out is null");
  *out = nullptr;
  int rc = tk_engine_preflight(cfg, class_table, class_len, pair_keys,
                               pair_keys_len, pair_vals, pair_vals_len, byte_id,
                               byte_id_len, vocab_keys, vocab_keys_len,
                               vocab_vals, vocab_vals_len, unsafe_bits,
                               unsafe_len);
  if (rc != TK_OK) return rc;
  if (cfg->needs_nfc && (!nfc_qc || nfc_qc_len < PLANE))
    return fail(TK_E_SHAPE, "needs_nfc requires the NFC quick-check table");
  if (cfg->ignore_merges && !vocab_blob && vocab_blob_len)
    return fail(TK_E_INVALID_ARG, "vocabulary blob is null");
  const uint64_t n_pairs = cfg->pair_count;
  // ranks are packed segment<<26|rank<<6|lane in 32 bits on the device
  // (a rank list whose products are 20-bit ids stays far below that), token
  // ids in 20 bits (the vocabulary value format already limits them to that)
  for (uint64_t i = 0; i < n_pairs; ++i) {
    if (pair_keys[i] == ~0ULL) continue;
    if ((pair_vals[i] >> 32) >= tk::MAX_MERGES)
      return fail(TK_E_SHAPE, "merge rank exceeds 2^20 - 2");
    if ((pair_vals[i] & 0xFFFFFFFFULL) >= (1u << 20) ||
        (pair_keys[i] >> 32) >= (1u << 20) ||
        (pair_keys[i] & 0xFFFFFFFFULL) >= (1u << 20))
      return fail(TK_E_SHAPE, "merge token id exceeds 2^20");
  }
  for (int b = 0; b < 256; ++b)
    if (byte_id[b] >= (1 << 20) - 1)
      return fail(TK_E_SHAPE, "byte token id exceeds 2^20 - 2");

  int ndev = 0;
  HIP_TRY(hipGetDeviceCount(&ndev));
  if (cfg->device_ordinal < 0 || cfg->device_ordinal >= ndev)
    return fail(TK_E_DEVICE, "device ordinal %d not present (%d devices)",
                cfg->device_ordinal, ndev);
  HIP_TRY(hipSetDevice(cfg->device_ordinal));
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, cfg->device_ordinal));
  std::string arch = prop.gcnArchName;
  const size_t colon = arch.find(':');
  if (colon != std::string::npos) arch = arch.substr(0, colon);
  if (cfg->expected_architecture && *cfg->expected_architecture &&
      arch != cfg->expected_architecture)
    return fail(TK_E_ARCH, "device architecture %s != expected %s",
                arch.c_str(), cfg->expected_architecture);

  tk_engine* e = new tk_engine();
  e->device = cfg->device_ordinal;
  e->cfg = *cfg;
  e->family = cfg->family ? cfg->family : "";
  e->sha = cfg->artifact_sha256 ? cfg->artifact_sha256 : "";
  e->cfg.family = e->family.c_str();
  e->cfg.artifact_sha256 = e->sha.c_str();
  e->cfg.expected_architecture = nullptr;
  e->arch = arch;
  {
    // a wait on another workgroup's published word gives up after WAIT_MS
    // (far above any launch: the longest measured, a guarded block merge
    // of a 32,000-space run, takes ~32 ms); another engine's kernels on
    // the same device can delay a predecessor's dispatch by a launch
    int khz = 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate,
                              cfg->device_ordinal) != hipSuccess || khz <= 0)
      khz = 100000;  // the 100 MHz counter of CDNA3 / CDNA4
    e->wait_ticks = (uint64_t)khz * WAIT_MS;
  }
  auto bail = [&](int code) {
    tk_engine_close(e);
    return code;
  };
  if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess ||
      hipStreamCreateWithFlags(&e->stream2, hipStreamNonBlocking) != hipSuccess ||
      hipStreamCreateWithFlags(&e->stream3, hipStreamNonBlocking) != hipSuccess)
    return bail(fail(TK_E_DEVICE, "hipStreamCreateWithFlags failed"));
  // join of the side stream into the engine stream (one device): no
  // system-scope fence
  if (hipEventCreateWithFlags(&e->ev_join, hipEventDisableTiming |
                                               hipEventDisableSystemFence) != hipSuccess ||
      hipEventCreateWithFlags(&e->ev_join3, hipEventDisableTiming |
                                                hipEventDisableSystemFence) != hipSuccess)
    return bail(fail(TK_E_DEVICE, "hipEventCreateWithFlags failed"));
  for (auto& ev : e->ev)
    // timing-only events: no system-scope fence between the stages
    if (hipEventCreateWithFlags(&ev, hipEventDisableSystemFence) != hipSuccess)
      return bail(fail(TK_E_DEVICE, "hipEventCreateWithFlags failed"));
  for (auto& pair : e->kev)
    for (auto& ev : pair)
      if (hipEventCreateWithFlags(&ev, hipEventDisableSystemFence) != hipSuccess)
        return bail(fail(TK_E_DEVICE, "hipEventCreateWithFlags failed"));
  // the device's copy of the static scratch array (the allocation-free
  // entry's workspace), looked up once per device with the device current
  {
    Workspace probe;
    if (carve(probe, nullptr, TK_NOALLOC_MAX_BYTES) > tk::SCRATCH_BYTES)
      return bail(fail(TK_E_INTERNAL, "scratch array smaller than its workspace"));
    if (tk::scratch_region(e->device, &e->scratch) != hipSuccess)
      return bail(fail(TK_E_DEVICE, "hipGetSymbolAddress of the scratch array failed"));
  }
  if (hipHostMalloc(reinterpret_cast<void**>(&e->host_ctrl),
                    tk::CTRL_WORDS * sizeof(uint32_t), hipHostMallocDefault) != hipSuccess)
    return bail(fail(TK_E_DEVICE, "hipHostMalloc failed"));
  {
    void* g = nullptr;
    if (hipHostMalloc(&g, tk::GATE_WORDS * sizeof(uint32_t),
                      hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess)
      return bail(fail(TK_E_DEVICE, "hipHostMalloc (gate) failed"));
    std::memset(g, 0, tk::GATE_WORDS * sizeof(uint32_t));
    e->gate = static_cast<volatile uint32_t*>(g);
    void* gd = nullptr;
    if (hipHostGetDevicePointer(&gd, g, 0) != hipSuccess)
      return bail(fail(TK_E_DEVICE, "hipHostGetDevicePointer failed"));
    e->gate_dev = static_cast<uint32_t*>(gd);
  }

  // interleave key/value so one 16-byte load reads a whole slot
  std::vector<ulonglong2> pairs(n_pairs);
  for (uint64_t i = 0; i < n_pairs; ++i) pairs[i] = {pair_keys[i], pair_vals[i]};
  std::vector<ulonglong2> vocab(cfg->vocab_count);
  for (uint64_t i = 0; i < cfg->vocab_count; ++i) vocab[i] = {vocab_keys[i], vocab_vals[i]};
  // direct table for the first merge level: both symbols still raw bytes
  std::vector<uint64_t> bp(65536, ~0ULL);
  for (int a = 0; a < 256; ++a)
    for (int b = 0; b < 256; ++b)
      if (byte_id[a] >= 0 && byte_id[b] >= 0)
        bp[(a << 8) | b] = host_pair_lookup(pair_keys, pair_vals, n_pairs,
                                            (uint32_t)byte_id[a], (uint32_t)byte_id[b]);

  auto up = [&](auto& buf, const void* src, size_t count) -> int {
    if (buf.alloc(count) != hipSuccess)
      return fail(TK_E_DEVICE, "hipMalloc of a %zu-entry table failed", count);
    if (count && hipMemcpy(buf.p, src, count * sizeof(*buf.p), hipMemcpyHostToDevice) != hipSuccess)
      return fail(TK_E_DEVICE, "table upload failed");
    return TK_OK;
  };
  if ((rc = up(e->cls, class_table, PLANE)) != TK_OK) return bail(rc);
  if ((rc = up(e->pairs, pairs.data(), pairs.size())) != TK_OK) return bail(rc);
  if ((rc = up(e->vocab, vocab.data(), vocab.size())) != TK_OK) return bail(rc);
  if ((rc = up(e->bytepair, bp.data(), bp.size())) != TK_OK) return bail(rc);
  if ((rc = up(e->byte_id, byte_id, 256)) != TK_OK) return bail(rc);
  const uint8_t zero = 0;
  if ((rc = up(e->blob, vocab_blob_len ? vocab_blob : &zero,
               vocab_blob_len ? vocab_blob_len : 1)) != TK_OK)
    return bail(rc);
  if (cfg->needs_nfc) {
    if ((rc = up(e->nfc, nfc_qc, PLANE)) != TK_OK) return bail(rc);
    e->host_nfc.assign(nfc_qc, nfc_qc + PLANE);
  }
  e->t.cls = e->cls.p;
  e->t.nfc = cfg->needs_nfc ? e->nfc.p : nullptr;
  e->t.pairs = e->pairs.p;
  e->t.pair_mask = n_pairs - 1;
  e->t.bytepair = e->bytepair.p;
  e->t.byte_id = e->byte_id.p;
  e->t.vocab = e->vocab.p;
  e->t.vocab_mask = cfg->vocab_count - 1;
  e->t.vocab_max_len = 0;
  for (uint64_t i = 0; i < cfg->vocab_count; ++i)
    if (vocab_keys[i] != ~0ULL)
      e->t.vocab_max_len = std::max(e->t.vocab_max_len,
                                    (uint32_t)((vocab_vals[i] >> 20) & 0x3FF));
  e->t.blob = e->blob.p;
  // Laguna runs the cl100k predicate inside the parts its newline-run
  // split makes; the split is a document-start pass ahead of k_pretok
  e->t.ruleset = cfg->ruleset == TK_RULESET_LAGUNA ? TK_RULESET_CL100K : cfg->ruleset;
  e->t.dmax = cfg->ruleset == TK_RULESET_R50K ? 0 : cfg->digits_max;
  e->added = tk::DevAdded{};
  e->added.newline_cuts = cfg->ruleset == TK_RULESET_LAGUNA ? 1 : 0;
  e->t.ignore_merges = cfg->ignore_merges ? 1 : 0;
  e->t.contractions = cfg->contractions ? 1 : 0;
  e->t.needs_nfc = cfg->needs_nfc ? 1 : 0;
  // Pieces over 512 bytes are cut and certified when every byte has an
  // initial id: from the segments' first / last-token events when every
  // merge rule that consumes a token ranks above every rule that produces
  // it (no bit set in unsafe_bits), else from every merge round of the
  // segments. A table that drops bytes merges them serially.
  bool monotone = true;
  for (size_t i = 0; i < unsafe_len / 4; ++i) monotone = monotone && unsafe_bits[i] == 0;
  bool all_bytes = true;
  for (int b = 0; b < 256; ++b) all_bytes = all_bytes && byte_id[b] >= 0;
  e->t.cert = !all_bytes ? 0 : monotone ? 1 : 2;
  e->t.all_bytes = all_bytes ? 1 : 0;
  e->t.ctab = nullptr;
  e->t.hot = nullptr;
  e->t.hot_k = 0;
  {
    // with the compact table every symbol the packed merge looks up (a
    // byte's id or a rule's product) is below 2^18
    bool small_ids = true;
    for (int b = 0; b < 256; ++b) small_ids = small_ids && byte_id[b] < (1 << 18);
    std::vector<uint64_t> ct;
    uint32_t bits = 0;
    PairEntries ent;
    if (small_ids && build_compact_pairs(pair_keys, pair_vals, n_pairs, ct, bits, &ent)) {
      if ((rc = up(e->ctab, ct.data(), ct.size())) != TK_OK) return bail(rc);
      e->t.ctab = e->ctab.p;
      e->t.cmask = (1ULL << bits) - 1;
      e->t.cbits = bits;
      // the hot pairs (probed only with TK_OPT_HOT_PAIRS)
      std::vector<uint64_t> ht;
      uint32_t hk = 0;
      if (build_hot_pairs(std::move(ent), ht, hk)) {
        if ((rc = up(e->hot, ht.data(), ht.size())) != TK_OK) return bail(rc);
        e->hot_k = hk;
      }
    }
  }
  e->t.unsafe = nullptr;
  e->t.unsafe_words = 0;
  if (!monotone) {
    if ((rc = up(e->unsafe, unsafe_bits, unsafe_len / 4)) != TK_OK) return bail(rc);
    e->t.unsafe = e->unsafe.p;
    e->t.unsafe_words = (uint32_t)(unsafe_len / 4);
  }
  if (hipDeviceSynchronize() != hipSuccess)
    return bail(fail(TK_E_DEVICE, "device synchronize after upload failed"));
  *out = e;
  return TK_OK;
}

void tk_engine_close(tk_engine* e) {
  if (!e) return;
  (void)hipSetDevice(e->device);
  if (e->stream) (void)hipStreamSynchronize(e->stream);
  for (auto& ev : e->ev)
    if (ev) (void)hipEventDestroy(ev);
  if (e->stream2) (void)hipStreamSynchronize(e->stream2);
  if (e->stream3) (void)hipStreamSynchronize(e->stream3);
  for (auto& pair : e->kev)
    for (auto& ev : pair)
      if (ev) (void)hipEventDestroy(ev);
  if (e->stream2) (void)hipStreamSynchronize(e->stream2);
  if (e->stream3) (void)hipStreamSynchronize(e->stream3);
  if (e->ev_join) (void)hipEventDestroy(e->ev_join);
  if (e->ev_join3) (void)hipEventDestroy(e->ev_join3);
  if (e->stream) (void)hipStreamDestroy(e->stream);
  if (e->stream2) (void)hipStreamDestroy(e->stream2);
  if (e->stream3) (void)hipStreamDestroy(e->stream3);
  if (e->host_ctrl) (void)hipHostFree(e->host_ctrl);
  if (e->gate) (void)hipHostFree(const_cast<uint32_t*>(e->gate));
  delete e;
}

int tk_engine_set_timing(tk_engine* e, int enabled) {
  if (!e) return fail(TK_E_INVALID_ARG, "engine is null");
  if (enabled < 0 || enabled > 2)
    return fail(TK_E_INVALID_ARG, "timing mode %d is not 0, 1 or 2", enabled);
  std::lock_guard<std::mutex> lk(e->mu);
  e->timing = enabled;
  return TK_OK;
}

int tk_engine_last_timing(const tk_engine* e, double* us, int n) {
  if (!e || !us) return fail(TK_E_INVALID_ARG, "null argument");
  int k = 0;
  for (; k < n && k < 8; ++k) us[k] = e->last_us[k];
  for (; k < n && k < 8 + TK_KERNELS; ++k) us[k] = e->last_kus[k - 8];
  return k;
}

int tk_engine_set_added(tk_engine* e, size_t n, const uint8_t* contents,
                        const uint64_t* offsets, const uint32_t* ids,
                        const uint8_t* flags) {
  if (!e) return fail(TK_E_INVALID_ARG, "engine is null");
  std::lock_guard<std::mutex> lk(e->mu);
  if (n > 0 && (!contents || !offsets || !ids || !flags))
    return fail(TK_E_INVALID_ARG, "null argument");
  if (n > (size_t)tk::ADDED_MAX_LITERALS)
    return fail(TK_E_UNSUPPORTED, "%zu added tokens (at most %d)", n,
                tk::ADDED_MAX_LITERALS);
  std::vector<std::string> raw, norm;
  for (size_t k = 0; k < n; ++k) {
    if (offsets[k + 1] < offsets[k])
      return fail(TK_E_INVALID_ARG, "offsets must be non-decreasing");
    const size_t len = offsets[k + 1] - offsets[k];
    const uint8_t* c = contents + offsets[k];
    if (len == 0 || len > (size_t)tk::ADDED_MAX_LEN)
      return fail(TK_E_UNSUPPORTED, "added token %zu has %zu bytes (1..%d)", k,
                  len, tk::ADDED_MAX_LEN);
    if (!utf8_ok(c, len))
      return fail(TK_E_INVALID_ARG, "added token %zu is not valid UTF-8", k);
    if (ids[k] == tk::INVALID_ID)
      return fail(TK_E_INVALID_ARG, "added token %zu has id 0xFFFFFFFF", k);
    if (flags[k] & (TK_ADDED_SINGLE_WORD | TK_ADDED_LSTRIP | TK_ADDED_RSTRIP))
      return fail(TK_E_UNSUPPORTED,
                  "added token %zu uses single_word / lstrip / rstrip", k);
    if (e->added.newline_cuts &&
        (c[0] == '\r' || c[0] == '\n' || c[len - 1] == '\r' || c[len - 1] == '\n'))
      return fail(TK_E_UNSUPPORTED,
                  "added token %zu begins or ends with CR or LF (the newline-run "
                  "split of this ruleset would see across it)", k);
    if ((flags[k] & TK_ADDED_NORMALIZED) && e->t.needs_nfc)
      return fail(TK_E_UNSUPPORTED,
                  "added token %zu is normalized=true and the family "
                  "normalizes: it would be matched on normalized segments", k);
    (flags[k] & TK_ADDED_NORMALIZED ? norm : raw)
        .emplace_back(reinterpret_cast<const char*>(c), len);
  }
  // HF extracts raw literals first and normalized ones in the segments
  // left over; with the identity normalizer one leftmost-longest pass gives
  // the same split exactly when no literal of one kind can overlap one of
  // the other
  for (const auto& x : raw)
    for (const auto& y : norm)
      if (can_overlap(x, y) || can_overlap(y, x))
        return fail(TK_E_UNSUPPORTED,
                    "a raw and a normalized added token can overlap");
  // trie: node 0 is the root
  std::vector<std::map<uint8_t, uint32_t>> kids(1);
  std::vector<uint32_t> term(1, 0);
  uint32_t lmax = 0;
  uint64_t gate[4] = {0, 0, 0, 0};
  std::vector<uint32_t> idv(n);
  std::vector<uint8_t> lens(n);
  for (size_t k = 0; k < n; ++k) {
    const uint8_t* c = contents + offsets[k];
    const uint32_t L = (uint32_t)(offsets[k + 1] - offsets[k]);
    uint32_t v = 0;
    for (uint32_t j = 0; j < L; ++j) {
      auto it = kids[v].find(c[j]);
      if (it == kids[v].end()) {
        const uint32_t u = (uint32_t)kids.size();
        kids[v][c[j]] = u;
        kids.emplace_back();
        term.push_back(0);
        v = u;
      } else {
        v = it->second;
      }
    }
    if (term[v]) return fail(TK_E_INVALID_ARG, "added token %zu is a duplicate", k);
    term[v] = (uint32_t)k + 1;
    idv[k] = ids[k];
    lens[k] = (uint8_t)L;
    lmax = std::max(lmax, L);
    gate[c[0] >> 6] |= 1ULL << (c[0] & 63);
  }
  if (kids.size() > tk::ADDED_MAX_NODES)
    return fail(TK_E_UNSUPPORTED, "added-token trie over %u nodes", tk::ADDED_MAX_NODES);
  // the edges in a hash table at most two thirds full (tk_device.h)
  size_t n_edges = kids.size() - 1;
  const uint32_t size = (uint32_t)std::max<size_t>(64, (3 * n_edges + 1) / 2 + 1);
  std::vector<uint64_t> tab(size, ~0ULL);
  for (size_t v = 0; v < kids.size(); ++v)
    for (const auto& kv : kids[v]) {
      const uint32_t key = ((uint32_t)v << 8) | kv.first, child = kv.second;
      uint32_t i = tk::added_slot(key, size);
      while (tab[i] != ~0ULL) i = i + 1 == size ? 0 : i + 1;
      tab[i] = ((uint64_t)key << 36) | ((uint64_t)child << 16) | term[child];
    }
  HIP_TRY(hipSetDevice(e->device));
  HIP_TRY(hipStreamSynchronize(e->stream));
  const int cuts = e->added.newline_cuts;
  e->added = tk::DevAdded{};
  e->added.newline_cuts = cuts;
  if (n == 0) return TK_OK;
  auto up = [&](auto& buf, const auto& v) -> int {
    if (buf.alloc(v.size()) != hipSuccess)
      return fail(TK_E_DEVICE, "hipMalloc of the added-token tables failed");
    if (hipMemcpy(buf.p, v.data(), v.size() * sizeof(v[0]), hipMemcpyHostToDevice) != hipSuccess)
      return fail(TK_E_DEVICE, "added-token table upload failed");
    return TK_OK;
  };
  int rc;
  if ((rc = up(e->lit_tab, tab)) != TK_OK) return rc;
  if ((rc = up(e->lit_len, lens)) != TK_OK) return rc;
  if ((rc = up(e->lit_id, idv)) != TK_OK) return rc;
  tk::DevAdded a{};
  a.tab = e->lit_tab.p;
  a.tab_size = size;
  a.len = e->lit_len.p;
  a.id = e->lit_id.p;
  for (int k = 0; k < 4; ++k) a.gate[k] = gate[k];
  a.lmax = lmax;
  a.n = (uint32_t)n;
  a.newline_cuts = cuts;
  e->added = a;
  return TK_OK;
}

int tk_engine_last_literals(const tk_engine* e, uint64_t* n) {
  if (!e || !n) return fail(TK_E_INVALID_ARG, "null argument");
  *n = e->last_literals;
  return TK_OK;
}

int tk_engine_set_option(tk_engine* e, int option, int64_t value) {
  if (!e) return fail(TK_E_INVALID_ARG, "engine is null");
  std::lock_guard<std::mutex> lk(e->mu);
  if (option == TK_OPT_COMPACT_PAIRS) {
    if (value != 0 && value != 1)
      return fail(TK_E_INVALID_ARG, "TK_OPT_COMPACT_PAIRS takes 0 or 1");
    e->t.ctab = value && e->ctab.p ? e->ctab.p : nullptr;
    return TK_OK;
  }
  if (option == TK_OPT_HOT_PAIRS) {
    if (value != 0 && value != 1)
      return fail(TK_E_INVALID_ARG, "TK_OPT_HOT_PAIRS takes 0 or 1");
    e->t.hot = value && e->hot.p ? e->hot.p : nullptr;
    e->t.hot_k = e->hot_k;
    return TK_OK;
  }
  if (option == TK_OPT_TIMED_KERNEL) {
    if (value < 0 || value >= TK_KERNELS)
      return fail(TK_E_INVALID_ARG, "TK_OPT_TIMED_KERNEL takes 0..%d", TK_KERNELS - 1);
    e->timed_kernel = (int)value;
    return TK_OK;
  }
  if (option == TK_OPT_REPAIR_WIDEN) {
    if (value < 0 || value > 64)
      return fail(TK_E_INVALID_ARG, "TK_OPT_REPAIR_WIDEN takes 0..64");
    e->repair_widen = (int)value;
    return TK_OK;
  }
  return fail(TK_E_INVALID_ARG, "unknown option %d", option);
}

int tk_engine_set_fault_marker(tk_engine* e, const uint8_t* marker, size_t len) {
  if (!e || (len && !marker)) return fail(TK_E_INVALID_ARG, "null argument");
  std::lock_guard<std::mutex> lk(e->mu);
  e->fault_marker.assign(reinterpret_cast<const char*>(marker), len);
  return TK_OK;
}

int tk_engine_last_stats(const tk_engine* e, uint64_t* out, int n) {
  if (!e || !out) return fail(TK_E_INVALID_ARG, "null argument");
  const uint64_t v[4] = {e->last_literals, e->last_nlong, e->last_big,
                         e->last_passes};
  int k = 0;
  for (; k < n && k < 4; ++k) out[k] = v[k];
  return k;
}

int tk_engine_driver_version(const tk_engine* e, int* version) {
  if (!e || !version) return fail(TK_E_INVALID_ARG, "null argument");
  HIP_TRY(hipDriverGetVersion(version));
  return TK_OK;
}

const char* tk_engine_delivery(const tk_engine* e) { return e ? "prebuilt" : ""; }
const char* tk_engine_architecture(const tk_engine* e) { return e ? e->arch.c_str() : ""; }

namespace {

// tk_engine_encode_device with the engine's lock held, the device current
// and a workspace that holds nbytes
static int device_encode(tk_engine* e, Workspace& ws, const void* d_text,
                         size_t nbytes, uint32_t flags, void* d_ids, size_t ids_cap,
                         size_t* n_ids, void* stream) {
  *n_ids = 0;
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : e->stream;
  const bool check = e->t.needs_nfc && !(flags & TK_FLAG_NORMALIZED);
  uint32_t st, total;
  tk::DevAdded docs;
  // the compaction writes straight into the caller's buffer
  int rc = run_pipeline(e, ws, static_cast<const uint8_t*>(d_text), nbytes,
                        nullptr, check, s, static_cast<uint32_t*>(d_ids),
                        ids_cap, &st, &total, doc_pass(e, flags, &docs));
  if (rc != TK_OK) return rc;
  if (st & tk::ST_UTF8) return fail(TK_E_UTF8, "input is not valid UTF-8");
  if (st & tk::ST_NFC) return fail(TK_E_NEEDS_NFC, "NFC quick check failed");
  if ((st & tk::ST_CAPACITY) || total > ids_cap)
    return fail(TK_E_CAPACITY, "%u ids exceed the %zu-id buffer", total, ids_cap);
  *n_ids = total;
  return TK_OK;
}

// the engine's own workspace, grown to hold nbytes
static int own_encode(tk_engine* e, const void* d_text, size_t nbytes,
                      uint32_t flags, void* d_ids, size_t ids_cap, size_t* n_ids,
                      void* stream) {
  *n_ids = 0;
  if (nbytes == 0) return TK_OK;
  HIP_TRY(hipSetDevice(e->device));
  int rc = ensure_workspace(e, nbytes, 0);
  if (rc != TK_OK) return rc;
  return device_encode(e, e->ws, d_text, nbytes, flags, d_ids, ids_cap, n_ids,
                       stream);
}

// One lock per device for the static scratch array: every engine on a
// device shares that device's copy of the array.
static std::mutex& scratch_lock(int device) {
  static std::mutex locks[64];
  return locks[device & 63];
}

}  // namespace

int tk_engine_encode_device(tk_engine* e, const void* d_text, size_t nbytes,
                            uint32_t flags, void* d_ids, size_t ids_cap,
                            size_t* n_ids, void* stream) {
  if (!e || !n_ids || (nbytes && (!d_text || !d_ids)))
    return fail(TK_E_INVALID_ARG, "null argument");
  std::lock_guard<std::mutex> lk(e->mu);
  return own_encode(e, d_text, nbytes, flags, d_ids, ids_cap, n_ids, stream);
}

int tk_engine_encode_device_noalloc(tk_engine* e, const void* d_text,
                                    size_t nbytes, uint32_t flags, void* d_ids,
                                    size_t ids_cap, size_t* n_ids,
                                    void* stream) {
  if (!e || !n_ids || (nbytes && (!d_text || !d_ids)))
    return fail(TK_E_INVALID_ARG, "null argument");
  *n_ids = 0;
  if (nbytes > TK_NOALLOC_MAX_BYTES)
    return fail(TK_E_CAPACITY,
                "input of %zu bytes exceeds the %u-byte limit of the "
                "allocation-free entry (use tk_engine_encode_device)",
                nbytes, (unsigned)TK_NOALLOC_MAX_BYTES);
  if (!e->scratch)
    return fail(TK_E_DEVICE, "the static scratch array has no device address");
  std::lock_guard<std::mutex> lk(e->mu);
  if (nbytes == 0) return TK_OK;
  std::lock_guard<std::mutex> sk(scratch_lock(e->device));
  HIP_TRY(hipSetDevice(e->device));
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : e->stream;
  // the entry waits for *n_ids (and reads host-mapped words mid-run), which
  // a stream under capture cannot do
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(s, &cap));
  if (cap != hipStreamCaptureStatusNone)
    return fail(TK_E_INVALID_ARG,
                "the stream is being captured: the entry synchronizes and "
                "cannot be recorded into a graph");
  // the workspace over the device's scratch array; the array keeps the last
  // call's contents, so the words that must start clear (the control slots
  // and the compaction status words) are cleared by a kernel first
  Workspace ws;
  carve(ws, e->scratch, TK_NOALLOC_MAX_BYTES);
  HIP_TRY(tk::launch_clear(ws.ctrl, 2 * tk::CTRL_WORDS, ws.cstat,
                           (uint32_t)ws.nblk, ws.nrun, 3 * (uint32_t)ws.tiles, s));
  return device_encode(e, ws, d_text, nbytes, flags, d_ids, ids_cap, n_ids,
                       stream);
}

int tk_engine_encode_seed(tk_engine* e, const void* d_text, size_t nbytes,
                          uint32_t flags, void* d_ids, size_t ids_cap,
                          uint32_t stride, void* d_points, size_t points_cap,
                          size_t* n_ids, size_t* n_points, void* stream) {
  if (!e || !n_ids || !n_points || (nbytes && (!d_text || !d_ids)))
    return fail(TK_E_INVALID_ARG, "null argument");
  if (stride == 0) return fail(TK_E_INVALID_ARG, "stride must be positive");
  std::lock_guard<std::mutex> lk(e->mu);
  *n_points = 0;
  int rc = own_encode(e, d_text, nbytes, flags, d_ids, ids_cap, n_ids, stream);
  if (rc != TK_OK || *n_ids == 0) return rc;
  // one checkpoint at every token index that is a multiple of the stride
  const size_t n = (*n_ids + stride - 1) / stride;
  if (n > points_cap || !d_points)
    return fail(TK_E_CAPACITY, "%zu checkpoints exceed the %zu-entry buffer", n,
                points_cap);
  if (n > 0x7FFFFFFFu) return fail(TK_E_CAPACITY, "too many checkpoints");
  const size_t nblk = (nbytes + tk::COMPACT_BLOCK - 1) / tk::COMPACT_BLOCK;
  if (e->seedc.n < nblk) HIP_TRY(e->seedc.alloc(nblk));
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : e->stream;
  // the pipeline's workspace still holds this encode's per-byte tokens
  // and the compaction's block prefix
  tk::DevWork w{};
  w.tok = e->ws.tok;
  w.blkprefix = e->ws.blkprefix;
  HIP_TRY(tk::launch_seed(w, static_cast<const uint8_t*>(d_text), (int64_t)nbytes,
                          (uint32_t)n, stride, e->seedc.p,
                          static_cast<uint64_t*>(d_points), s));
  HIP_TRY(hipStreamSynchronize(s));
  *n_points = n;
  return TK_OK;
}

namespace {
// the injected fault of a host-buffer call (tk_engine_set_fault_marker)
static bool injected_fault(const tk_engine* e, const uint8_t* data, size_t n) {
  const std::string& m = e->fault_marker;
  if (m.empty() || n < m.size()) return false;
  const uint8_t* end = data + n;
  return std::search(data, end, m.begin(), m.end(),
                     [](uint8_t a, char b) { return a == (uint8_t)b; }) != end;
}

}  // namespace

int tk_engine_encode_seed_host(tk_engine* e, const uint8_t* text, size_t nbytes,
                               uint32_t flags, uint32_t* ids, size_t ids_cap,
                               uint32_t stride, uint64_t* points,
                               size_t points_cap, size_t* n_ids,
                               size_t* n_points) {
  if (!e || !n_ids || !n_points || (nbytes && (!text || !ids)))
    return fail(TK_E_INVALID_ARG, "null argument");
  if (stride == 0) return fail(TK_E_INVALID_ARG, "stride must be positive");
  std::lock_guard<std::mutex> lk(e->mu);
  *n_ids = 0;
  *n_points = 0;
  if (nbytes == 0) return TK_OK;
  HIP_TRY(hipSetDevice(e->device));
  int rc = ensure_workspace(e, nbytes, 0);
  if (rc != TK_OK) return rc;
  hipStream_t s = e->stream;
  if ((rc = stage_in(e, e->ws.text, text, nbytes, s)) != TK_OK) return rc;
  HostOut o;
  if ((rc = host_out(e, ids, ids_cap, &o)) != TK_OK) return rc;
  const bool check = e->t.needs_nfc && !(flags & TK_FLAG_NORMALIZED);
  uint32_t st, total;
  tk::DevAdded docs;
  rc = run_pipeline(e, e->ws, e->ws.text, nbytes, nullptr, check, s, o.dev,
                    o.cap, &st, &total, doc_pass(e, flags, &docs));
  if (rc != TK_OK) return rc;
  if (st & tk::ST_UTF8) return fail(TK_E_UTF8, "input is not valid UTF-8");
  if (st & tk::ST_NFC) return fail(TK_E_NEEDS_NFC, "NFC quick check failed");
  if (total > ids_cap)
    return fail(TK_E_CAPACITY, "%u ids exceed the %zu-id buffer", total, ids_cap);
  if (injected_fault(e, text, nbytes)) return fail(TK_E_INTERNAL, "injected fault");
  const size_t n = total ? (total + stride - 1) / stride : 0;
  if (n > points_cap || (n && !points))
    return fail(TK_E_CAPACITY, "%zu checkpoints exceed the %zu-entry buffer", n,
                points_cap);
  if (n) {
    // the checkpoints into engine-owned device memory, behind the ids
    const size_t nblk = (nbytes + tk::COMPACT_BLOCK - 1) / tk::COMPACT_BLOCK;
    if (e->seedc.n < nblk) HIP_TRY(e->seedc.alloc(nblk));
    if (e->seedp.n < 3 * n) HIP_TRY(e->seedp.alloc(3 * n));
    tk::DevWork w{};
    w.tok = e->ws.tok;
    w.blkprefix = e->ws.blkprefix;
    HIP_TRY(tk::launch_seed(w, e->ws.text, (int64_t)nbytes, (uint32_t)n, stride,
                            e->seedc.p, e->seedp.p, s));
  }
  if (n)
    HIP_TRY(hipMemcpyAsync(points, e->seedp.p, 3 * n * sizeof(uint64_t),
                           hipMemcpyDeviceToHost, s));
  ids_from_staging(e, o, ids, total);
  if (n) HIP_TRY(hipStreamSynchronize(s));
  *n_ids = total;
  *n_points = n;
  return TK_OK;
}

int tk_engine_encode(tk_engine* e, const uint8_t* text, size_t nbytes,
                     uint32_t flags, uint32_t* ids, size_t ids_cap,
                     size_t* n_ids) {
  if (!e || !n_ids || (nbytes && (!text || !ids)))
    return fail(TK_E_INVALID_ARG, "null argument");
  std::lock_guard<std::mutex> lk(e->mu);
  *n_ids = 0;
  if (nbytes == 0) return TK_OK;
  HIP_TRY(hipSetDevice(e->device));
  int rc = ensure_workspace(e, nbytes, 0);
  if (rc != TK_OK) return rc;
  hipStream_t s = e->stream;
  using clk = std::chrono::steady_clock;
  const auto h0 = clk::now();
  if ((rc = stage_in(e, e->ws.text, text, nbytes, s)) != TK_OK) return rc;
  HostOut o;
  if ((rc = host_out(e, ids, ids_cap, &o)) != TK_OK) return rc;
  const auto h1 = clk::now();
  const bool check = e->t.needs_nfc && !(flags & TK_FLAG_NORMALIZED);
  uint32_t st, total;
  tk::DevAdded docs;
  rc = run_pipeline(e, e->ws, e->ws.text, nbytes, nullptr, check, s, o.dev,
                    o.cap, &st, &total, doc_pass(e, flags, &docs));
  const auto h2 = clk::now();
  if (rc != TK_OK) return rc;
  if (st & tk::ST_UTF8) return fail(TK_E_UTF8, "input is not valid UTF-8");
  if (st & tk::ST_NFC) return fail(TK_E_NEEDS_NFC, "NFC quick check failed");
  if (total > ids_cap) return fail(TK_E_CAPACITY, "%u ids exceed the %zu-id buffer", total, ids_cap);
  if (injected_fault(e, text, nbytes)) return fail(TK_E_INTERNAL, "injected fault");
  ids_from_staging(e, o, ids, total);
  const auto h3 = clk::now();
  auto us = [](clk::duration d) {
    return std::chrono::duration<double, std::micro>(d).count();
  };
  e->last_us[5] = us(h1 - h0);
  e->last_us[6] = us(h2 - h1);
  e->last_us[7] = us(h3 - h2);
  *n_ids = total;
  return TK_OK;
}

namespace {

// The documents end to end into dst, by the copy threads in claims of
// STAGE_CHUNK bytes of the joined range (a claim copies the parts of the
// documents it covers); offs: the documents' offsets, offs.back() bytes.
static void gather_docs(tk_engine* e, uint8_t* dst, const uint8_t* const* docs,
                        const std::vector<uint64_t>& offs) {
  const size_t nb = offs.back();
  auto part = [&](size_t lo, size_t hi) {
    // the document holding byte lo (past any empty ones)
    size_t d = (size_t)(std::upper_bound(offs.begin(), offs.end(), (uint64_t)lo) -
                        offs.begin()) - 1;
    while (lo < hi) {
      const size_t end = std::min<size_t>(hi, offs[d + 1]);
      if (end > lo) std::memcpy(dst + lo, docs[d] + (lo - offs[d]), end - lo);
      lo = std::max(lo, end);
      ++d;
    }
  };
  if (nb <= STAGE_SMALL) {
    part(0, nb);
    return;
  }
  copy_pool(e)->run((nb + STAGE_CHUNK - 1) / STAGE_CHUNK, [&](size_t k) {
    const size_t lo = k * STAGE_CHUNK;
    part(lo, std::min(nb, lo + STAGE_CHUNK));
  });
}

// The batch entries' body, under the engine's lock: `joined` holds the
// documents' bytes in host memory (the caller's buffer, or the pinned
// staging that gather_docs filled).
static int encode_batch_locked(tk_engine* e, const uint8_t* joined,
                               const uint64_t* doc_offsets, size_t n_docs,
                               uint32_t flags, uint32_t* ids, size_t ids_cap,
                               uint64_t* row_offsets, int32_t* row_status) {
  const size_t nb = n_docs ? doc_offsets[n_docs] : 0;
  for (size_t d = 0; d < n_docs; ++d) {
    if (doc_offsets[d] > doc_offsets[d + 1])
      return fail(TK_E_INVALID_ARG, "doc_offsets must be non-decreasing");
    row_status[d] = TK_OK;
  }
  if (doc_offsets[0] != 0) return fail(TK_E_INVALID_ARG, "doc_offsets[0] must be 0");
  for (size_t d = 0; d <= n_docs; ++d) row_offsets[d] = 0;
  if (nb == 0) return TK_OK;
  if (!joined || !ids) return fail(TK_E_INVALID_ARG, "null argument");
  HIP_TRY(hipSetDevice(e->device));
  int rc = ensure_workspace(e, nb, n_docs);
  if (rc != TK_OK) return rc;
  hipStream_t s = e->stream;
  // forced piece starts at every document head (gpu.rs:644-652): the mask
  // is built on the device from the offsets
  if ((rc = stage_in(e, e->ws.text, joined, nb, s)) != TK_OK) return rc;
  // (the offsets cross from page-locked memory: one plain DMA)
  std::memcpy(e->offs_pin.p, doc_offsets, (n_docs + 1) * 8);
  HIP_TRY(hipMemcpyAsync(e->docoffs.p, e->offs_pin.p, (n_docs + 1) * 8, hipMemcpyHostToDevice, s));
  HIP_TRY(tk::launch_doc_mask(e->ws.docmask, (int64_t)((nb + 63) / 64 + 2),
                              e->docoffs.p, (uint32_t)n_docs, (int64_t)nb, s));
  HostOut o;
  if ((rc = host_out(e, ids, ids_cap, &o)) != TK_OK) return rc;
  const bool check = e->t.needs_nfc && !(flags & TK_FLAG_NORMALIZED);
  uint32_t st, total;
  tk::DevAdded docs;
  const RowsOut ro{e->docoffs.p, (uint32_t)n_docs,
                   reinterpret_cast<uint64_t*>(e->rows_pin.dev)};
  rc = run_pipeline(e, e->ws, e->ws.text, nb, e->ws.docmask, check, s,
                    o.dev, o.cap, &st, &total, doc_pass(e, flags, &docs), &ro);
  if (rc != TK_OK) return rc;
  if (total > ids_cap) return fail(TK_E_CAPACITY, "%u ids exceed the %zu-id buffer", total, ids_cap);
  // a batch holding a poisoned document fails as a whole, as a device
  // guard trip would
  for (size_t d = 0; d < n_docs && !e->fault_marker.empty(); ++d)
    if (injected_fault(e, joined + doc_offsets[d], doc_offsets[d + 1] - doc_offsets[d])) {
      HIP_TRY(hipStreamSynchronize(s));
      return fail(TK_E_INTERNAL, "injected fault (document %zu)", d);
    }
  // (the pipeline's sync has made the row offsets visible here)
  std::memcpy(row_offsets, e->rows_pin.p, (n_docs + 1) * 8);
  ids_from_staging(e, o, ids, total);
  if (st & (tk::ST_UTF8 | tk::ST_NFC)) {
    // find the rows that failed; their ids are dropped, the others stand
    std::vector<uint32_t> keep;
    keep.reserve(total);
    std::vector<uint64_t> rows(row_offsets, row_offsets + n_docs + 1);
    uint64_t acc = 0;
    for (size_t d = 0; d < n_docs; ++d) {
      const uint8_t* doc = joined + doc_offsets[d];
      const size_t len = doc_offsets[d + 1] - doc_offsets[d];
      int rs = TK_OK;
      if ((st & tk::ST_UTF8) && !host_utf8_ok(doc, len)) rs = TK_E_UTF8;
      else if ((st & tk::ST_NFC) && check && !host_nfc_ok(e->host_nfc, doc, len))
        rs = TK_E_NEEDS_NFC;
      row_status[d] = rs;
      row_offsets[d] = acc;
      if (rs == TK_OK)
        for (uint64_t k = rows[d]; k < rows[d + 1]; ++k) keep.push_back(ids[k]);
      acc = keep.size();
    }
    row_offsets[n_docs] = acc;
    std::memcpy(ids, keep.data(), keep.size() * 4);
  }
  return TK_OK;
}

}  // namespace

int tk_engine_encode_batch(tk_engine* e, const uint8_t* joined,
                           const uint64_t* doc_offsets, size_t n_docs,
                           uint32_t flags, uint32_t* ids, size_t ids_cap,
                           uint64_t* row_offsets, int32_t* row_status) {
  if (!e || !doc_offsets || !row_offsets || !row_status)
    return fail(TK_E_INVALID_ARG, "null argument");
  std::lock_guard<std::mutex> lk(e->mu);
  return encode_batch_locked(e, joined, doc_offsets, n_docs, flags, ids, ids_cap,
                             row_offsets, row_status);
}

int tk_engine_encode_batch_docs(tk_engine* e, const uint8_t* const* docs,
                                const size_t* doc_lens, size_t n_docs,
                                uint32_t flags, uint32_t* ids, size_t ids_cap,
                                uint64_t* row_offsets, int32_t* row_status) {
  if (!e || !row_offsets || !row_status || (n_docs && (!docs || !doc_lens)))
    return fail(TK_E_INVALID_ARG, "null argument");
  std::lock_guard<std::mutex> lk(e->mu);
  std::vector<uint64_t> offs(n_docs + 1, 0);
  for (size_t d = 0; d < n_docs; ++d) {
    if (doc_lens[d] && !docs[d]) return fail(TK_E_INVALID_ARG, "document %zu is null", d);
    offs[d + 1] = offs[d] + doc_lens[d];
  }
  const uint8_t* joined = nullptr;
  if (offs[n_docs]) {
    // (the pinned staging, already the size stage_in would make it; its
    // bytes then go to the device in one transfer, as a page-locked
    // request does)
    HIP_TRY(hipSetDevice(e->device));
    HIP_TRY(e->pin_in.ensure(std::max((size_t)offs[n_docs], e->ws.cap) + 64));
    gather_docs(e, e->pin_in.p, docs, offs);
    joined = e->pin_in.p;
  }
  return encode_batch_locked(e, joined, offs.data(), n_docs, flags, ids, ids_cap,
                             row_offsets, row_status);
}

}  // extern "C"
