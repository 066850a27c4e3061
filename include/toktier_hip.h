/*
 * toktier_hip.h -- C-ABI of the MI355X (gfx950) fresh-encode engine.
 *
 * One engine = one tokenizer family on one GPU: UTF-8 bytes in, byte-level
 * BPE token ids out, bit-identical to a from-scratch Hugging Face
 * `tokenizers` encode of the same text (add_special_tokens=False).
 *
 * The entry points replace the reference's Rust GPU engine surface:
 *   tk_engine_preflight  <- NativePrebuiltGpu::preflight
 *                           (crates/toktier-routing-core/src/gpu.rs:1383-1404,
 *                            shape rules validate_tables gpu.rs:1642-1679)
 *   tk_engine_open       <- NativePrebuiltGpu::new / Executor::new
 *                           (gpu.rs:1406-1442, :248-344)
 *   tk_engine_encode     <- NativeGpuEngine::encode_ids
 *                           (runtime.rs:76-82; gpu.rs:1446-1461, :500-600)
 *   tk_engine_encode_batch <- NativeGpuEngine::encode_batch_ids
 *                           (gpu.rs:1463-1546, Executor::encode_batch :605-750)
 *   tk_engine_encode_batch_docs <- the same, with the documents as the
 *                           reference passes them (texts: &[&str],
 *                           gpu.rs:1463): separate buffers
 *   tk_engine_set_added  <- AddedTokenFrontend construction and the
 *                           router's added-token check ahead of the GPU
 *                           (src/toktier/frontend/added.py:316-375, scan
 *                           :503-533, assemble :544-555;
 *                           runtime.rs:527-536, :641-662): the literals are
 *                           extracted on the device instead of routing
 *                           the whole input to the CPU reference
 *   tk_engine_last_literals <- the R_INPUT_ADDED_TOKEN ledger fact
 *                           (runtime.rs:648-654), as a count
 *   tk_engine_delivery   <- NativeGpuEngine::delivery (runtime.rs:81)
 *   tk_engine_close      <- Drop of the engine / CUDA driver RAII
 *                           (crates/toktier-cuda-driver/src/lib.rs:424-457)
 *   tk_last_error        <- NativeRuntimeError / CudaError message
 *                           (runtime.rs:58-72; cuda-driver lib.rs:31-49)
 * The table arguments are the reference's kernel-input ABI unchanged
 * (src/toktier/kernels/bpe_tables.py:1-30): pair_keys/pair_vals (u64,
 * splitmix64 open addressing), byte_id (i32[256]), vocab_keys/vocab_vals/
 * vocab_blob (FNV-1a-64 whole-piece hash), unsafe_bits (u32 bitmap), class
 * table (u8[0x110000], P=0 L=1 N=2 S=3). The engine re-packs them into its
 * own device layout at open.
 *
 * Threading: calls on one engine serialize on an internal mutex (the
 * reference's Mutex<Executor>, gpu.rs:1361, :1457-1460). Errors: every
 * entry returns a TK_* status; on failure no ids are produced and
 * tk_last_error() (thread-local) describes the failure.
 */
#ifndef TOKTIER_HIP_H
#define TOKTIER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TK_ABI_VERSION 1u

/* rulesets (the reference names: gpu.rs:40-62; r50k is new) */
#define TK_RULESET_CL100K 0 /* Qwen2 / Llama-3 split (digits_max 1 or 3) */
#define TK_RULESET_R50K 1   /* GPT-2 split */
#define TK_RULESET_LAGUNA 2 /* Laguna-S-2.1: (?:\r?\n)+ split MergedWithNext,
                               then the cl100k split (digits_max 1)
                               (pretok_kernel.cu:76-86) */
#define TK_RULESET_DEEPSEEK 3 /* DeepSeek V3 / V4: Split stages \p{N}{1,3},
                                 CJK-range runs, then the main pattern
                                 (pretok_classes_deepseek.v1.meta.json
                                 "patterns"; digits_max 3, the seven-class
                                 table, contractions 0) */
#define TK_RULESET_O200K 4 /* gpt-oss: o200k_base (options.rs O200k row;
                              kernel_families.v1.json gpt_oss_120b: digits_max
                              3, contractions; the rows with contractions
                              false and digits_max 1 too), the seven-class
                              table P U L C N S M of class table o200k_v4 */
#define TK_RULESET_KIMI 5  /* Kimi K3: [\p{Han}]+ first, the o200k letter
                              alternatives without Han, \p{N}{1,3}, a
                              punctuation tail without '/' (conversion.py
                              KIMI_PATTERN; kernel_families.v1.json kimi_k3:
                              digits_max 3, contractions), the ten-class
                              table of kimi_v1 (P U L C N S M HL HN HP) */

/* status codes */
#define TK_OK 0
#define TK_E_INVALID_ARG (-1) /* null pointer, bad config field */
#define TK_E_SHAPE (-2)       /* table shape rules (gpu.rs:1642-1679) */
#define TK_E_DEVICE (-3)      /* HIP runtime failure */
#define TK_E_ARCH (-4)        /* device is not the expected architecture */
#define TK_E_UTF8 (-5)        /* input is not valid UTF-8 */
#define TK_E_NEEDS_NFC (-6)   /* NFC quick check failed: normalize, retry */
#define TK_E_CAPACITY (-7)    /* caller's id buffer too small / input too big */
#define TK_E_INTERNAL (-8)
#define TK_E_UNSUPPORTED (-9) /* an added-token table this engine refuses */

/* tk_engine_encode flags */
#define TK_FLAG_NORMALIZED 1u /* caller already applied the family's NFC */
#define TK_FLAG_NO_ADDED 2u   /* do not extract added-token literals: the
                                 caller already split them out (the text is
                                 one segment between literals) */

/* added-token flags (tokenizer.json "added_tokens" fields) */
#define TK_ADDED_SPECIAL 1u
#define TK_ADDED_SINGLE_WORD 2u
#define TK_ADDED_LSTRIP 4u
#define TK_ADDED_RSTRIP 8u
#define TK_ADDED_NORMALIZED 16u

typedef struct tk_engine tk_engine;

/* NativePrebuiltGpuConfig (gpu.rs:22-38) minus the fatbin digest fields */
typedef struct tk_config {
  uint32_t abi_version;        /* TK_ABI_VERSION */
  int32_t device_ordinal;
  int32_t ruleset;             /* TK_RULESET_* */
  int32_t digits_max;          /* cl100k: 1 (Qwen) or 3 (Llama); r50k: 0;
                                  kimi: 3 */
  int32_t contractions;        /* 1, or 0 for deepseek (its pattern has
                                  no contraction alternative); o200k: 1 or
                                  0 (the rows without the suffix) */
  int32_t needs_nfc;           /* family declares an NFC normalizer */
  int32_t ignore_merges;       /* whole-piece vocabulary hit first */
  uint64_t pair_count;         /* slots in pair_keys (power of two) */
  uint64_t vocab_count;        /* slots in vocab_keys (power of two) */
  const char* family;          /* label only */
  const char* artifact_sha256; /* label only */
  const char* expected_architecture; /* "gfx950" or NULL for any */
} tk_config;

/* Device-free validation of the config and table shapes. Sizes are bytes. */
int tk_engine_preflight(const tk_config* cfg,
                        const uint8_t* class_table, size_t class_len,
                        const uint64_t* pair_keys, size_t pair_keys_len,
                        const uint64_t* pair_vals, size_t pair_vals_len,
                        const int32_t* byte_id, size_t byte_id_len,
                        const uint64_t* vocab_keys, size_t vocab_keys_len,
                        const uint64_t* vocab_vals, size_t vocab_vals_len,
                        const uint32_t* unsafe_bits, size_t unsafe_len);

/* Opens the device, uploads the tables. nfc_qc (u8[0x110000]) is needed
 * only when cfg->needs_nfc. */
int tk_engine_open(const tk_config* cfg,
                   const uint8_t* class_table, size_t class_len,
                   const uint64_t* pair_keys, size_t pair_keys_len,
                   const uint64_t* pair_vals, size_t pair_vals_len,
                   const int32_t* byte_id, size_t byte_id_len,
                   const uint64_t* vocab_keys, size_t vocab_keys_len,
                   const uint64_t* vocab_vals, size_t vocab_vals_len,
                   const uint8_t* vocab_blob, size_t vocab_blob_len,
                   const uint32_t* unsafe_bits, size_t unsafe_len,
                   const uint8_t* nfc_qc, size_t nfc_qc_len,
                   tk_engine** out);

void tk_engine_close(tk_engine* engine);

/* One request: host UTF-8 in, host ids out. ids_cap >= nbytes always
 * suffices (a token covers at least one byte). Pageable request bytes are
 * copied into the engine's pinned staging by its copy threads and sent in
 * one transfer; page-locked ones (hipHostMalloc) are sent directly. The
 * compaction kernel writes the ids straight into a page-locked, 4-byte
 * aligned ids buffer (the serving configuration: no transfer command, no
 * host copy), or into the engine's pinned staging, from which the copy
 * threads fill a pageable one. After a failure (*n_ids == 0) the first
 * ids_cap entries of a page-locked ids buffer hold no defined values; a
 * pageable one is left as it was. The same holds for the batch and the
 * host-buffer seed entries. */
int tk_engine_encode(tk_engine* engine, const uint8_t* text, size_t nbytes,
                     uint32_t flags, uint32_t* ids, size_t ids_cap,
                     size_t* n_ids);

/* A batch: documents concatenated in `joined`, document d spans
 * [doc_offsets[d], doc_offsets[d+1]) bytes. Row d's ids land in
 * ids[row_offsets[d] .. row_offsets[d+1]); each row equals
 * tk_engine_encode of that document alone. row_status[d] is TK_OK or the
 * row's own error (e.g. TK_E_NEEDS_NFC); rows with an error are empty. */
int tk_engine_encode_batch(tk_engine* engine, const uint8_t* joined,
                           const uint64_t* doc_offsets, size_t n_docs,
                           uint32_t flags, uint32_t* ids, size_t ids_cap,
                           uint64_t* row_offsets, int32_t* row_status);

/* The same batch with document d in its own buffer docs[d] of doc_lens[d]
 * bytes (a null pointer only where the length is 0): the engine's copy
 * threads gather the documents into its pinned staging, so the caller
 * joins nothing. Rows, status and errors as tk_engine_encode_batch. */
int tk_engine_encode_batch_docs(tk_engine* engine, const uint8_t* const* docs,
                                const size_t* doc_lens, size_t n_docs,
                                uint32_t flags, uint32_t* ids, size_t ids_cap,
                                uint64_t* row_offsets, int32_t* row_status);

/* Device-resident form (no host copies): d_text and d_ids are device
 * pointers on the engine's device; `stream` is a hipStream_t or NULL for
 * the engine's own stream. Blocks until *n_ids is known. The ids are
 * compacted straight into d_ids; after a failure (*n_ids == 0) its first
 * ids_cap entries hold no defined values. */
int tk_engine_encode_device(tk_engine* engine, const void* d_text,
                            size_t nbytes, uint32_t flags, void* d_ids,
                            size_t ids_cap, size_t* n_ids, void* stream);

/* Allocation-free form of tk_engine_encode_device. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid hipMalloc). Like every entry here it
 * waits for *n_ids, so it cannot be recorded into a HIP graph: on a stream
 * under capture it returns TK_E_INVALID_ARG and runs nothing. It calls no
 * hipMalloc / hipFree and no allocating library
 * routine: the per-request workspace is carved from a static device array
 * (one copy per device, about 96 MiB, held until the process ends) instead
 * of the engine's own workspace; the tables are the ones tk_engine_open
 * uploaded. Same arguments, results and errors as tk_engine_encode_device,
 * for inputs of at most TK_NOALLOC_MAX_BYTES bytes (larger inputs:
 * TK_E_CAPACITY, nothing run). Every engine on a device shares that
 * device's array, which keeps the last call's contents (each call clears
 * what must start at zero): calls that would overlap on one device are
 * serialized by a process-wide lock per device, and work that used the
 * array from outside this library would race with them. */
#define TK_NOALLOC_MAX_BYTES 1048576u
int tk_engine_encode_device_noalloc(tk_engine* engine, const void* d_text,
                                    size_t nbytes, uint32_t flags, void* d_ids,
                                    size_t ids_cap, size_t* n_ids,
                                    void* stream);

/* Session seed: tk_engine_encode_device plus the sparse span checkpoints
 * the session store adopts with the ids (replaces the span bridge of the
 * GPU seed: crates/toktier-store-core/src/tail.rs:17-31 SpanCheckpoint,
 * :173-205 build_span_checkpoints; SPAN_CHECKPOINT_STRIDE = 4096 there).
 * For every token index k * stride below *n_ids, d_points[3k .. 3k+2]
 * (device, uint64) receive: the token's first byte offset, the offset of
 * the first byte of the character holding it, and that character's index
 * in the text. *n_points = ceil(*n_ids / stride); TK_E_CAPACITY when that
 * exceeds points_cap (the ids are valid then). The tokens close over the
 * text by construction: the byte offsets are the prefix sums of the
 * tokens' byte lengths. */
int tk_engine_encode_seed(tk_engine* engine, const void* d_text,
                          size_t nbytes, uint32_t flags, void* d_ids,
                          size_t ids_cap, uint32_t stride, void* d_points,
                          size_t points_cap, size_t* n_ids, size_t* n_points,
                          void* stream);

/* tk_engine_encode_seed with host buffers: the text is read from host
 * memory through the engine's pinned staging, the ids and the checkpoints
 * (three uint64 each, as above) are written to host memory; the device
 * buffers are the engine's own. Replaces the same reference call as
 * tk_engine_encode_seed, for hosts that keep the session store in host
 * memory (crates/toktier-store-core/src/tail.rs:173-205). */
int tk_engine_encode_seed_host(tk_engine* engine, const uint8_t* text,
                               size_t nbytes, uint32_t flags, uint32_t* ids,
                               size_t ids_cap, uint32_t stride,
                               uint64_t* points, size_t points_cap,
                               size_t* n_ids, size_t* n_points);

/* Added tokens of the artifact (tokenizer.json "added_tokens", in artifact
 * order): literal k is contents[offsets[k] .. offsets[k+1]) (UTF-8, 1..255
 * bytes, all distinct), its id ids[k], its flags flags[k] (TK_ADDED_*).
 * Every later encode (unless TK_FLAG_NO_ADDED) first splits the text at
 * the literals the way HF tokenizers 0.22.2 does (leftmost match, the
 * longest at that position, scanning on after it), emits each literal's
 * id, and encodes the text between literals segment by segment (each
 * segment is pretokenized as a document of its own). n == 0 removes the
 * table. TK_E_UNSUPPORTED: a literal with single_word / lstrip / rstrip,
 * a normalized literal when the family normalizes (NFC), normalized and
 * raw literals that can overlap (HF extracts them in two passes), or, for
 * TK_RULESET_LAGUNA, a literal that begins or ends with CR or LF. */
int tk_engine_set_added(tk_engine* engine, size_t n, const uint8_t* contents,
                        const uint64_t* offsets, const uint32_t* ids,
                        const uint8_t* flags);

/* Literals extracted by the last encode on this engine. */
int tk_engine_last_literals(const tk_engine* engine, uint64_t* n);

/* Facts of the last encode on this engine (the reference's per-execution
 * ledger facts, runtime.rs:641-697, as counts): [0] added-token literals
 * extracted, [1] pieces over 64 bytes, [2] pieces over 512 bytes (cut and
 * certified), [3] certification repair passes (each removes the cuts whose
 * certificate failed and redoes the joined segments). Returns the number
 * of values written (<= n). */
#define TK_STAT_LITERALS 0
#define TK_STAT_LONG 1
#define TK_STAT_BIG 2
#define TK_STAT_REPAIRS 3
int tk_engine_last_stats(const tk_engine* engine, uint64_t* out, int n);

/* HIP driver version of the engine's device (hipDriverGetVersion; the
 * reference driver surface's driver_version(), cuda-driver lib.rs:51-86),
 * for the route's driver floor. */
int tk_engine_driver_version(const tk_engine* engine, int* version);

const char* tk_engine_delivery(const tk_engine* engine);     /* "prebuilt" */
const char* tk_engine_architecture(const tk_engine* engine); /* "gfx950" */

/* Device times (microseconds) of the last encode on this engine, from HIP
 * events taken by the dispatches themselves. Mode 1 (every stage): [0]
 * pretokenize and piece listing, [1] short-piece BPE, [2] the time the
 * long-piece BPE (run beside the short-piece BPE) went past it, [3]
 * compaction, [4] total, and [8 + k] the own duration of kernel k
 * (TK_KERNEL_*; 0 when the call did not launch it). Mode 2 (least
 * disturbance): [1] the own duration of the one kernel TK_OPT_TIMED_KERNEL
 * names (default TK_KERNEL_BPE_PACK; 0 when the call did not launch it),
 * the others 0. Mode 0 (default): nothing is recorded. Host wall times of
 * the last tk_engine_encode, in every mode: [5] the request bytes into
 * device memory, [6] the pipeline up to the ids being final in device
 * memory, [7] the ids into the caller's buffer. Returns the number of
 * values written (<= n, at most 8 + TK_KERNELS). */
#define TK_KERNEL_PRETOK 0       /* k_pretok: pretokenize, list the pieces */
#define TK_KERNEL_BPE_PACK 1     /* k_bpe_pack: pieces of up to 128 bytes */
#define TK_KERNEL_COMPACT 2      /* k_compact: ids compacted */
#define TK_KERNEL_BPE_ROWS 3     /* k_bpe_rows: pieces of 129-256 bytes */
#define TK_KERNEL_LONG_WINDOWS 4 /* k_long_windows: cuts of pieces > 512 B */
#define TK_KERNEL_ADDED 5        /* k_added: added-token literal split */
#define TK_KERNELS 6
int tk_engine_set_timing(tk_engine* engine, int mode);
int tk_engine_last_timing(const tk_engine* engine, double* us, int n);

/* Engine options (no reference counterpart). TK_OPT_COMPACT_PAIRS: 1
 * (default) probe the compact pair table the engine builds at open when
 * the artifact fits it, 0 probe the boundary-format table (the reference's
 * splitmix64 open addressing) on every path. Returns TK_OK, or
 * TK_E_INVALID_ARG for an unknown option or value. */
#define TK_OPT_COMPACT_PAIRS 1
/* TK_OPT_REPAIR_WIDEN: pieces over 512 bytes are cut into segments and
 * every cut certified; a failed cut is dropped and its segments redone, one
 * repair pass after another. From this pass on (default 4; 1..64) each
 * failed cut also drops its 4^(p - value + 1) nearest cuts on each side
 * inside its piece, so a cascade of failures (each drop exposing the next,
 * as in periodic runs) ends within a few passes. 0: every piece over 512
 * bytes is merged whole by a workgroup, with no cut (the path of tables
 * that drop bytes). */
#define TK_OPT_REPAIR_WIDEN 2
/* TK_OPT_TIMED_KERNEL: the TK_KERNEL_* timing mode 2 times. */
#define TK_OPT_TIMED_KERNEL 3
/* TK_OPT_HOT_PAIRS: 1 makes the merge kernels of pieces of 65..256 bytes
 * probe a 16 KB copy of the lowest-ranked rules in LDS before the pair
 * table in HBM (when the engine built the compact table); 0 (default) the
 * table only. */
#define TK_OPT_HOT_PAIRS 4
int tk_engine_set_option(tk_engine* engine, int option, int64_t value);

/* Test-only fault injection (no counterpart in the reference; the hook its
 * tests drive with a stand-in encoder, gpu.rs:1828-1854, made a property
 * of the engine so the error contract can be driven through the real
 * path): while a marker is set (len > 0; len 0 clears it), a call of
 * tk_engine_encode, tk_engine_encode_batch or tk_engine_encode_seed_host
 * whose input holds the marker bytes runs its pipeline, then fails as a
 * whole with TK_E_INTERNAL and writes no ids (a batch fails when any of
 * its documents holds it, as a device guard trip fails the batch). */
int tk_engine_set_fault_marker(tk_engine* engine, const uint8_t* marker,
                               size_t len);

/* Thread-local description of the last failure on this thread. */
const char* tk_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* TOKTIER_HIP_H */
