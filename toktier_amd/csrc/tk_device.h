// tk_device.h -- device-side data layout and stage launchers of the gfx950
// fresh-encode engine (internal to libtoktier_hip; not part of the C-ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tk {

constexpr uint32_t INVALID_ID = 0xFFFFFFFFu;
constexpr uint32_t RANK_INF = 0xFFFFFFFFu;
// pair keys inside a wave are (63 - segment start)<<26 | rank<<6 | lane
constexpr uint32_t MAX_MERGES = (1u << 20) - 1;  // ranks < 2^20 - 1

// status word bits (device -> host)
constexpr uint32_t ST_UTF8 = 1u;     // invalid UTF-8 seen
constexpr uint32_t ST_NFC = 2u;      // NFC quick check failed
constexpr uint32_t ST_LONGOVF = 4u;  // long-piece list overflow (internal)
constexpr uint32_t ST_CAPACITY = 8u;  // more ids than the output holds
constexpr uint32_t ST_STALL = 16u;    // compaction look-back timed out (internal)
constexpr uint32_t ST_STALL_PRETOK = 32u;  // a pretokenize tile's look-back
                                           // (digit run, o200k state) timed out
constexpr uint32_t ST_ROUNDS = 64u;   // a workgroup merge ran past its round
                                      // bound (internal)

// Compact pair table: 16-byte buckets of two u64 slots, two candidate
// buckets per pair (cuckoo placement), so a lookup is two independent
// 16-byte loads and no probe chain; at a load of about 0.6 the table is a
// quarter of the boundary table's size and stays in an XCD's L2.
// The pair key (left, right < 2^18) goes through a bijection of 36 bits
// (one Feistel round: left << 18 | right ^ f(left), where f is a 24-bit
// multiply, full rate on the vector ALU, folded onto itself). Its low
// `bits` bits are the first bucket, the rest the tag; the second bucket is
// the first XOR a hash of the tag. Slot = tag<<38 | second<<37 | rank<<18
// | id, so (bucket, slot) names its key exactly; an empty slot is all ones,
// which no tag reaches.
constexpr uint32_t CTAB_MIN_BITS = 12;
constexpr uint32_t CTAB_MAX_BITS = 22;
__host__ __device__ __forceinline__ uint32_t pair_round(uint32_t x, uint32_t c) {
  const uint32_t p = (x & 0x3FFFFu) * c;
  return (p ^ (p >> 16)) & 0x3FFFFu;
}
__host__ __device__ __forceinline__ uint64_t pair_perm(uint32_t l, uint32_t r) {
  const uint32_t b = r ^ pair_round(l, 0x9E3779u);
  return ((uint64_t)(l & 0x3FFFFu) << 18) | (b & 0x3FFFFu);
}
// second bucket of a key with first bucket b1 and tag (< 2^24)
__host__ __device__ __forceinline__ uint32_t pair_alt(uint32_t b1, uint32_t tag,
                                                      uint32_t bits) {
  const uint32_t h = (tag & 0xFFFFFFu) * 0xC2B2AFu;  // a 24-bit multiply
  return (b1 ^ (h >> (32 - bits))) & ((1u << bits) - 1);
}

// Device copies of the family tables, in the engine's own layout.
struct DevTables {
  const uint8_t* cls;          // [0x110000] P/L/N/S (deepseek: O L M N PS WS CRLF;
                               // o200k: P U L C N S M; kimi: + HL HN HP)
  const uint8_t* nfc;          // [0x110000] quick-check values or nullptr
  const ulonglong2* pairs;     // interleaved {key, val} merge hash slots
  uint64_t pair_mask;
  const uint64_t* bytepair;    // [65536] rank<<32|id for two raw bytes, ~0 none
  const int32_t* byte_id;      // [256]
  const ulonglong2* vocab;     // interleaved {fnv key, val} vocabulary slots
  uint64_t vocab_mask;
  uint32_t vocab_max_len;      // bytes of the longest vocabulary entry
  const uint8_t* blob;         // vocabulary bytes
  int32_t ruleset;             // 0 cl100k, 1 r50k, 3 deepseek, 4 o200k, 5 kimi
  int32_t dmax;                // digit group width (cl100k)
  int32_t ignore_merges;
  int32_t needs_nfc;
  int32_t contractions;        // o200k: the contraction suffix is on
  int32_t cert;                // long pieces over 512 bytes: 0 merged
                               // serially (a byte without an id); 1 cut and
                               // certified from first / last-token events
                               // (every rule that consumes a token ranks
                               // above the rule that makes it); 2 cut and
                               // certified from every merge round (any table)
  int32_t all_bytes;           // every byte has an id (no dropped bytes)
  const uint32_t* unsafe;      // unsafe-rank bitmap or nullptr
  uint32_t unsafe_words;
  const uint64_t* ctab;        // compact pair table or nullptr
  uint64_t cmask;              // buckets - 1
  uint32_t cbits;              // log2(buckets)
  // hot pairs: the rules of rank < hot_k in the compact table's layout with
  // HOT_BITS buckets (HOT_BYTES), copied into LDS by the kernels that probe
  // it before the table in HBM; nullptr: none
  const uint64_t* hot;
  uint32_t hot_k;
};

// The hot-pair table: 2^HOT_BITS buckets of 16 bytes (16 KB), the compact
// table's bijection, bucket pair and slot layout with a 26-bit tag. An
// empty slot is all ones; its rank field (2^19 - 1) is never below hot_k,
// which is how a probe tells it from a rule.
constexpr uint32_t HOT_BITS = 10;
constexpr uint32_t HOT_BYTES = 16u << HOT_BITS;

// length classes of the packed short-piece BPE (see pack_slot)
constexpr int PACK_CLASSES = 13;

// Per-request device buffers (sized by capacity).
struct DevWork {
  const uint8_t* text;   // nb bytes (+ padding readable)
  int64_t nb;
  const uint64_t* docmask;  // doc-start bits or nullptr (single document)
  int check_nfc;            // run the quick check this call
  uint64_t* starts;      // piece-start bits, one word per 64 bytes (+2)
  uint32_t* tok;         // per byte: token id at the byte where it starts,
                         // INVALID_ID elsewhere
  int32_t* nx;           // long-piece scratch (per byte)
  int32_t* pv;
  uint64_t* heap;        // long-piece heap scratch (3 per byte)
  uint32_t* longlist;    // (start, end) pairs
  uint32_t* longcount;   // [1]
  uint32_t long_cap;     // capacity of longlist in pairs
  uint32_t* status;      // ctrl[0]; ctrl[1] = total ids
  uint32_t* blkcount;    // per compaction block
  uint32_t* blkprefix;   // exclusive prefix, [nblk + 1]
  uint64_t* cstat;       // [nblk] compaction status words (look-back)
  uint32_t* out;         // compacted ids
  uint32_t out_cap;      // capacity of out in ids
  // long-piece segmentation (one bit / slot per byte)
  uint64_t* inlong;      // bytes of pieces over 64 bytes
  uint64_t* cuts;        // candidate segment starts inside long pieces
  uint64_t* failm;       // cuts whose certificate failed this pass
  uint64_t* hfirst;      // first-token merge events, at the segment start
                         // (cert 2: every merge round, see HR_FIRST)
  uint64_t* hlast;       // last-token merge events, at the segment start
  uint32_t* hmeta;       // event counts (first | last << 16; cert 2: rounds)
  uint32_t* seglist;     // segments that fit no grid window
  uint32_t* segcount;    // ctrl[3]
  uint32_t seg_cap;
  uint32_t* wlist;       // a repair pass's windows: v << 1 | (phase 0 too)
  uint32_t* wcount;      // ctrl[12]
  uint32_t wlist_cap;
  uint32_t* nfail;       // this certify pass's failed cuts (ctrl[4] / [8])
  uint32_t* nfail_prev;  // a device-side repair pass: the previous pass's
                         // count (the pass runs only when it is not 0);
                         // nullptr for the first pass and every other stage
  uint32_t* npass;       // device-side repair passes that ran (ctrl)
  uint64_t* dirty_cur;   // repair pass: words (64 bytes) to redo, 1 bit each
  uint64_t* dirty_next;  // words marked by the current certify pass
  // packed short-piece BPE: the piece starts of each length class, one
  // list per class and segment (pack_seg_list), in the order k_pretok's
  // tiles took their room
  uint32_t* plist;
  uint32_t* pseg;        // ctrl + CTRL_PSEG: per segment, k_bpe_pack's unit
                         // counter and the pieces listed per class
  uint32_t* nbig;        // queued pieces over WIDE_MAX bytes (ctrl)
  uint32_t* nrows;       // queued pieces of 129..256 bytes (ctrl)
  uint32_t* rowq;        // k_bpe_rows' piece counters, one per XCD (ctrl)
  uint32_t* vlist;       // the grid windows with long-piece bytes (k_win_list)
  uint32_t* vcount;      // their number (ctrl)
  uint32_t* nwide;       // queued pieces of 257..WIDE_MAX bytes (ctrl)
  uint32_t* prepdone;    // k_bpe_pack waves done with the long pieces (ctrl)
  uint32_t* gate;        // GATE_WORDS in host memory, or nullptr
  uint32_t seq;          // call number written to gate[GATE_SEQ]
  // bound of every wait on another workgroup's published word, in ticks
  // of the device's constant-rate real-time counter (wall_clock64)
  uint64_t wait_ticks;
  // added-token literals (nullptr when the call extracts none): a literal
  // [s, e) marks s in lits and s+1..e-1 in litb, and s and e as document
  // starts; its bytes form no piece, and its id is written at tok[s]
  uint64_t* lits;
  uint64_t* litb;
  uint32_t* nlit;        // literals extracted (ctrl)
  // per tile of k_pretok: the digit run at its end (call tag << 32 | whole
  // tile | N characters), or nullptr
  uint64_t* nrun;
  // (o200k) per tile of k_pretok: two words of its automaton function /
  // the state after it (o2_publish)
  uint64_t* ostate;
  // per-call clearing done by k_pretok for the stages after it
  uint32_t* ctrl_next;   // the other control slot (used by the next call)
  int64_t clear_words;   // inlong / failm words
  int64_t clear_dwords;  // dirty_next words
};

// A merge-round record of a segment (cert 2): rank << 32 | flags | product
// id. HR_FIRST / HR_LAST: the round changed the segment's first / last
// token (into the product). A round merges one pair, or every leftmost
// non-overlapping occurrence of a rank whose product no earlier rule
// consumes.
constexpr uint64_t HR_FIRST = 1ull << 31, HR_LAST = 1ull << 30;

// ctrl word layout (device -> host)
// (the words of segment x of the piece lists start at CTRL_PSEG + x *
// CTRL_PSEG_STRIDE: k_bpe_pack's unit counter, then on the next 128-byte
// line the pieces listed per class, at CTRL_PSEG_COUNT + class)
constexpr int CTRL_STATUS = 0, CTRL_TOTAL = 1, CTRL_LONG = 2, CTRL_SEG = 3,
              CTRL_FAIL = 4, CTRL_BIG = 5, CTRL_NLIT = 6, CTRL_PASS = 7,
              CTRL_FAIL2 = 8, CTRL_PREP = 9, CTRL_WIDE = 10, CTRL_ROWS = 11,
              CTRL_WIN = 12, CTRL_ROWQ = 16,  // (ROWQ: PACK_XCDS words)
              CTRL_VLIST = 24,
              CTRL_PSEG = 64, CTRL_PSEG_STRIDE = 64,
              CTRL_PSEG_COUNT = 32, CTRL_WORDS = CTRL_PSEG + 8 * CTRL_PSEG_STRIDE;
// gate words in host memory: k_bpe_pack writes GATE_NLONG / GATE_NROWS /
// GATE_NWIDE / GATE_BIG and then GATE_SEQ (the host learns, while the packed merge runs,
// whether the side streams' long-piece stages have any work), k_compact's
// last block writes the request's outcome (status, id count, failed cuts)
// and then GATE_DONE, so no copy is needed to read it
constexpr int GATE_SEQ = 0, GATE_BIG = 1, GATE_STATUS = 2, GATE_TOTAL = 3,
              GATE_FAIL = 4, GATE_DONE = 5, GATE_NLONG = 6, GATE_NLIT = 7,
              GATE_PASS = 8, GATE_NWIDE = 9, GATE_NROWS = 10, GATE_WORDS = 16;

// Added-token literals on the device: the trie over their bytes, stored as
// one hash table of its edges. Slot = key << 36 | child << 16 | term, key =
// parent node << 8 | byte (node 0 is the root), term = the literal ending
// at the child plus one (0: none); an empty slot is all ones (no node
// reaches 2^20 - 1). A key's first slot is (hash(key) * size) >> 32, then
// the next ones in order, wrapping (the table is at most two thirds full).
struct DevAdded {
  const uint64_t* tab;    // trie edges
  uint32_t tab_size;      // slots
  const uint8_t* len;     // literal bytes
  const uint32_t* id;     // literal token id
  uint64_t gate[4];       // the literals' first bytes (bit b of word b/64)
  uint32_t lmax;          // longest literal, bytes (1..255)
  uint32_t n;             // literals (0: none to extract this call)
  int newline_cuts;       // Laguna stage 0: a document start where each
                          // (?:\r?\n)+ run begins (split MergedWithNext)
};
constexpr int ADDED_MAX_LEN = 255;
constexpr int ADDED_MAX_LITERALS = 65535;
constexpr uint32_t ADDED_MAX_NODES = (1u << 20) - 2;
constexpr int ADDED_BLOCK_BYTES = 4096;  // bytes (64 mask words) per block
// tables up to these sizes are copied to LDS by the blocks that see a
// literal's first byte (larger ones are read from HBM)
constexpr int ADDED_TAB_LDS = 1536;   // edge slots (12 KiB)
constexpr int ADDED_LEN_LDS = 1024;   // literal lengths
__host__ __device__ __forceinline__ uint32_t added_slot(uint32_t key,
                                                        uint32_t size) {
  return (uint32_t)(((uint64_t)(key * 0x9E3779B1u) * size) >> 32);
}
// packed short-piece BPE: grid of k_bpe_pack, seven waves on every SIMD
// (blocks of four waves, 256 CUs); the eighth wave slot is left to the
// side streams' long-piece kernels, which run beside it
constexpr int PACK_BLOCKS = 1792;
// k_bpe_pack merges the queued pieces of 65..128 bytes itself when at most
// this many pieces over 64 bytes are queued; else k_bpe_rows does
constexpr int PACK_ROWS_MAX = 8192;
// The piece lists come in PACK_XCDS segments: segment x holds the pieces of
// the k_pretok tiles b with b % PACK_XCDS == x (those of one XCD: workgroups
// go to the XCDs in turn), and the k_bpe_pack blocks of the same residue
// merge them, each XCD's units handed out by a counter of its own
constexpr int PACK_XCDS = 8;
static_assert(CTRL_WORDS == CTRL_PSEG + PACK_XCDS * CTRL_PSEG_STRIDE,
              "one control line per segment");
static_assert(CTRL_ROWQ + PACK_XCDS <= CTRL_VLIST, "row counters before the window list's");
static_assert(CTRL_VLIST < CTRL_PSEG, "the window count before the segment lines");
// slots (lanes per piece) of the length classes, and the shortest piece of
// each class: class c holds pieces of pack_lmin(c)..pack_slot(c) bytes
__host__ __device__ constexpr int pack_slot(int c) {
  return c <= 6 ? c + 2 : c == 7 ? 10 : c == 8 ? 12 : c == 9 ? 16
       : c == 10 ? 21 : c == 11 ? 32 : 64;
}
// Classes of up to PACK_LANE_MAX bytes are merged one piece per lane (64
// pieces per work unit, each merged serially by its lane); up to
// PACK_GROUP_MAX bytes one piece per group of four lanes, 8 positions per
// lane (16 pieces per unit); longer ones lane per byte, 64 / slot pieces at
// a time (pieces per unit 64 / slot; lanes per piece recorded as 0).
constexpr int PACK_LANE_MAX = 16;
constexpr int PACK_GROUP_MAX = 32;
__host__ __device__ constexpr bool pack_lane(int c) {
  return pack_slot(c) <= PACK_LANE_MAX;
}
// lanes per piece of class c (0: lane per byte)
__host__ __device__ constexpr int pack_lanes(int c) {
  return pack_lane(c) ? 1 : pack_slot(c) <= PACK_GROUP_MAX ? 4 : 0;
}
// pieces per work unit, and a multiplier m with (lane * m) >> 12 == lane /
// pack_slot(c) for every lane < 64 (the lane-per-byte path, also taken by
// tables without the lane and group paths)
__host__ __device__ constexpr int pack_per_unit(int c) {
  return pack_lanes(c) ? 64 / pack_lanes(c) : 64 / pack_slot(c);
}
__host__ __device__ constexpr int pack_magic(int c) {
  return (4096 + pack_slot(c) - 1) / pack_slot(c);
}
__host__ __device__ constexpr int pack_lmin(int c) {
  return c <= 7 ? c + 2 : pack_slot(c - 1) + 1;
}

constexpr int PRETOK_TPB = 256;
constexpr int PT_TILE = 2816;  // bytes per k_pretok block (44 start words)
// k_pretok blocks: the start words 0..nwin+1 (nwin = ceil(nb / 64))
__host__ __device__ inline int64_t pretok_tiles(int64_t nb) {
  return (((nb + 63) / 64 + 2) * 64 + PT_TILE - 1) / PT_TILE;
}
// Room in the piece lists: a tile holds at most pack_local_cap(c) pieces of
// class c (every piece of pack_lmin(c) or more bytes that starts in it), so
// the lists take PT_LOCAL_SLOTS words per tile. Segment x's lists follow
// those of the segments before it; its class c list starts pack_local_off(c)
// words per tile of the segment into them.
__host__ __device__ constexpr int pack_local_cap(int c) {
  return PT_TILE / pack_lmin(c) + 1;
}
__host__ __device__ constexpr int pack_local_off(int c) {
  return c == 0 ? 0 : pack_local_off(c - 1) + pack_local_cap(c - 1);
}
constexpr int PT_LOCAL_SLOTS = pack_local_off(PACK_CLASSES);
// tiles of segment x, and of the segments before it, out of ntile
__host__ __device__ inline uint32_t pack_seg_tiles(uint32_t ntile, int x) {
  return ntile > (uint32_t)x ? (ntile - (uint32_t)x + PACK_XCDS - 1) / PACK_XCDS : 0u;
}
__host__ __device__ inline uint32_t pack_seg_first(uint32_t ntile, int x) {
  uint32_t n = 0;
  for (int y = 0; y < x; ++y) n += pack_seg_tiles(ntile, y);
  return n;
}
// start of segment x's class c list (local_off = pack_local_off(c))
__host__ __device__ inline uint32_t pack_seg_list(uint32_t ntile, int x,
                                                  uint32_t local_off) {
  return pack_seg_first(ntile, x) * (uint32_t)PT_LOCAL_SLOTS +
         pack_seg_tiles(ntile, x) * local_off;
}
constexpr int COMPACT_TPB = 256;
constexpr int COMPACT_PER_THREAD = 32;
constexpr int COMPACT_BLOCK = COMPACT_TPB * COMPACT_PER_THREAD;  // 8192

// start / stop: optional timing events taken from the start of the stage's
// first dispatch / the end of its last one
hipError_t launch_pretok(const DevTables& t, const DevWork& w, hipStream_t s,
                         hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
hipError_t launch_bpe_pack(const DevTables& t, const DevWork& w, hipStream_t s,
                           hipEvent_t start, hipEvent_t stop);
hipError_t launch_bpe_rows(const DevTables& t, const DevWork& w, hipStream_t s,
                           uint32_t nlong, hipEvent_t start = nullptr,
                           hipEvent_t stop = nullptr);
hipError_t launch_bpe_wide(const DevTables& t, const DevWork& w, hipStream_t s,
                           hipEvent_t stop, uint32_t nlong);
hipError_t launch_long_windows(const DevTables& t, const DevWork& w,
                               hipStream_t s, hipEvent_t start = nullptr,
                               hipEvent_t stop = nullptr);
hipError_t launch_long_segments(const DevTables& t, const DevWork& w, hipStream_t s);
// the first pass's listed segments (at most 64 bytes each)
hipError_t launch_seg_lists(const DevTables& t, const DevWork& w, hipStream_t s);
// pieces over WIDE_MAX bytes merged whole, a workgroup each (tables that
// drop bytes: no cut certification)
hipError_t launch_long_block(const DevTables& t, const DevWork& w, hipStream_t s);
hipError_t launch_certify(const DevTables& t, const DevWork& w, int all,
                          hipStream_t s, hipEvent_t stop = nullptr);
// (width > 0: each failed cut also drops its `width` nearest cuts on each
// side inside its piece, k_fail_widen, first)
hipError_t launch_apply_fail(const DevWork& w, hipStream_t s, uint32_t width);
// A repair pass's merges (after launch_apply_fail): the windows of the dirty
// words and the segments that fit no window, listed by k_seg_scan and
// merged together by k_repair_merge, then the segments over WIDE_MAX bytes
// (k_seg_block).
hipError_t launch_repair_segments(const DevTables& t, const DevWork& w, hipStream_t s);
// the first repair pass that widens the failed cuts (TK_OPT_REPAIR_WIDEN),
// and the width of pass p >= it: 4^(p - first + 1), capped
constexpr int REPAIR_WIDEN = 4;
__host__ __device__ constexpr uint32_t repair_width(int p, int first) {
  return first <= 0 || p < first ? 0u
         : (p - first + 1) >= 15 ? (1u << 30)
                                 : (1u << (2 * (p - first + 1)));
}
hipError_t launch_compact(const DevWork& w, hipStream_t s, uint32_t tag,
                          hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
// k_added: the literal split of the request into w.docmask (read-write;
// the document starts the caller marked, if any, are read from host_dm, a
// different buffer, and kept)
// session-seed checkpoints of the encode just compacted from w.tok (see
// k_seed_points); ccount: (nb + COMPACT_BLOCK - 1) / COMPACT_BLOCK words
hipError_t launch_seed(const DevWork& w, const uint8_t* text, int64_t nb,
                       uint32_t n_points, uint32_t stride, uint32_t* ccount,
                       uint64_t* pts, hipStream_t s);
hipError_t launch_added(const DevAdded& a, const DevWork& w,
                        const uint64_t* host_dm, hipStream_t s,
                        hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
hipError_t launch_doc_offsets(const DevWork& w, const uint64_t* doc_offsets,
                              uint32_t n_docs, uint64_t* row_offsets,
                              hipStream_t s);
// the document-start mask of a batch (nwords words) from its offsets
// (n_docs + 1 of them, non-decreasing) in device memory
hipError_t launch_doc_mask(uint64_t* mask, int64_t nwords,
                           const uint64_t* doc_offsets, uint32_t n_docs,
                           int64_t nb, hipStream_t s);

// The allocation-free entry (tk_engine_encode_device_noalloc) carves its
// workspace out of a static device array of SCRATCH_BYTES, one copy per
// device, held until the process ends. scratch_region returns that copy's
// device address on `device` (looked up once per device, with the device
// made current; the array's name in host code is not a device address).
constexpr size_t SCRATCH_BYTES = (size_t)96 << 20;
hipError_t scratch_region(int device, uint8_t** p);
// clears a[0..na) and b[0..nb) with a kernel (no memset node, so the call
// stays capturable)
hipError_t launch_clear(uint32_t* a, uint32_t na, uint64_t* b, uint32_t nb,
                        uint64_t* c, uint32_t nc, hipStream_t s);

}  // namespace tk
