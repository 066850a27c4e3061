/* toktier_oracle.h -- CPU restatement of the fresh-encode path.
 * TEST INFRASTRUCTURE ONLY (parity checker); see toktier_oracle.c. */
#ifndef TOKTIER_ORACLE_H
#define TOKTIER_ORACLE_H
#include <stdint.h>

#define TKO_RULESET_CL100K 0
#define TKO_RULESET_R50K 1
#define TKO_RULESET_LAGUNA 2
#define TKO_RULESET_DEEPSEEK 3
#define TKO_RULESET_O200K 4
#define TKO_RULESET_KIMI 5

#define TKO_E_UTF8 (-1)
#define TKO_E_NOMEM (-2)
#define TKO_E_NEEDS_NFC (-3)
#define TKO_E_CAP (-4)
#define TKO_E_CLASS (-5)  /* a class value the ruleset does not define */

typedef struct tko_tables {
  const uint8_t* cls;          /* 0x110000 class bytes (P/L/N/S; deepseek: O L M N PS WS
                                  CRLF; o200k: P U L C N S M; kimi: + HL HN HP) */
  const uint64_t* pair_keys;
  const uint64_t* pair_vals;
  uint64_t pair_count;         /* power of two */
  const int32_t* byte_id;      /* [256] */
  const uint64_t* vocab_keys;
  const uint64_t* vocab_vals;
  uint64_t vocab_count;        /* power of two */
  const uint8_t* vocab_blob;
  const uint8_t* nfc_qc;       /* 0x110000 or NULL */
  int32_t ruleset;
  int32_t digits_max;
  int32_t ignore_merges;
  int32_t needs_nfc;
  int32_t contractions;         /* o200k / kimi: the (?i:'s|...) suffix */
} tko_tables;

int64_t tko_utf8_decode(const uint8_t* s, int64_t nb, int32_t* cp, int64_t* bo);
int64_t tko_pretokenize(const tko_tables* t, const uint8_t* s, int64_t nb,
                        int64_t* starts);
int64_t tko_bpe(const tko_tables* t, const uint8_t* s, int64_t m, uint32_t* out);
int tko_nfc_qc(const tko_tables* t, const uint8_t* s, int64_t nb);
int64_t tko_encode(const tko_tables* t, const uint8_t* s, int64_t nb,
                   uint32_t* out, int64_t cap);

/* added-token literals: literal k is blob[offsets[k] .. offsets[k+1]) */
typedef struct tko_added {
  const uint8_t* blob;
  const uint64_t* offsets;  /* n + 1 */
  const uint32_t* ids;
  int64_t n;
} tko_added;
int64_t tko_encode_added(const tko_tables* t, const tko_added* a,
                         const uint8_t* s, int64_t nb, uint32_t* out,
                         int64_t cap);
#endif
