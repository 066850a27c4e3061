// tk_device.h -- device-side data layout and stage launchers of the gfx950
// fresh-encode engine (internal to libtoktier_hip; not part of the C-ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tk {

constexpr uint32_t INVALID_ID = 0xFFFFFFFFu;
constexpr uint32_t RANK_INF = 0xFFFFFFFFu;
// ranks are packed as rank<<6|lane into 32 bits inside a wave
constexpr uint32_t MAX_MERGES = 1u << 25;

// status word bits (device -> host)
constexpr uint32_t ST_UTF8 = 1u;     // invalid UTF-8 seen
constexpr uint32_t ST_NFC = 2u;      // NFC quick check failed
constexpr uint32_t ST_LONGOVF = 4u;  // long-piece list overflow (internal)

// Device copies of the family tables, in the engine's own layout.
struct DevTables {
  const uint8_t* cls;          // [0x110000] P/L/N/S
  const uint8_t* nfc;          // [0x110000] quick-check values or nullptr
  const ulonglong2* pairs;     // interleaved {key, val} merge hash slots
  uint64_t pair_mask;
  const uint64_t* bytepair;    // [65536] rank<<32|id for two raw bytes, ~0 none
  const int32_t* byte_id;      // [256]
  const ulonglong2* vocab;     // interleaved {fnv key, val} vocabulary slots
  uint64_t vocab_mask;
  const uint8_t* blob;         // vocabulary bytes
  int32_t ruleset;             // 0 cl100k, 1 r50k
  int32_t dmax;                // digit group width (cl100k)
  int32_t ignore_merges;
  int32_t needs_nfc;
};

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
  uint32_t* status;      // [1]
  uint32_t* blkcount;    // per compaction block
  uint32_t* blkprefix;   // exclusive prefix, [nblk + 1]
  uint32_t* out;         // compacted ids
};

constexpr int PRETOK_BYTES_PER_THREAD = 16;
constexpr int PRETOK_TPB = 256;
constexpr int COMPACT_TPB = 256;
constexpr int COMPACT_PER_THREAD = 16;
constexpr int COMPACT_BLOCK = COMPACT_TPB * COMPACT_PER_THREAD;  // 4096

hipError_t launch_pretok(const DevTables& t, const DevWork& w, hipStream_t s);
hipError_t launch_bpe_small(const DevTables& t, const DevWork& w,
                            hipStream_t s);
hipError_t launch_bpe_queue(const DevTables& t, const DevWork& w,
                            hipStream_t s);
hipError_t launch_bpe_long(const DevTables& t, const DevWork& w,
                           hipStream_t s);
hipError_t launch_compact(const DevWork& w, hipStream_t s);
hipError_t launch_doc_offsets(const DevWork& w, const uint64_t* doc_offsets,
                              uint32_t n_docs, uint64_t* row_offsets,
                              hipStream_t s);

}  // namespace tk
