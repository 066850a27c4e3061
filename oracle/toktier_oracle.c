/*
 * toktier_oracle.c -- CPU restatement of the GPU fresh-encode path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the parity tests,
 * the smoke entry and the bench's cpu_baseline leg compare the HIP engine
 * against. Nothing on the product path links, loads or calls it.
 *
 * It restates, in plain sequential C:
 *   - strict UTF-8 decoding (src/toktier/kernels/pretok_kernel.cu:363-407:
 *     truncated sequences, F8-FF leads, overlong forms, surrogates and
 *     values above U+10FFFF are invalid);
 *   - the family split regexes as a left-to-right alternation matcher, one
 *     alternative at a time in pattern order, with the greedy/backtracking
 *     outcome of each alternative written out:
 *       cl100k (Qwen2 / Llama-3):
 *         (?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}{1,K}
 *         | ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+
 *       (crates/toktier-gigatoken-core/src/pretokenize/options.rs:125,:131;
 *        K = digits_max, kernel_families.v1.json:104-117)
 *       laguna (Laguna-S-2.1): (?:\r?\n)+ split MergedWithNext first,
 *         then the cl100k pattern (K = 1) inside each part
 *       r50k (GPT-2):
 *         's|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+
 *         |\s+(?!\S)|\s+
 *       (options.rs:118; crates/.../pretokenize/fast/r50k.rs:1-2)
 *       deepseek (DeepSeek V3 / V4): three Split(Isolated) stages in
 *         order, \p{N}{1,3}, then [\u4e00-\u9fa5\u3040-\u309f\u30a0-\u30ff]+,
 *         then [ascii punct][A-Za-z]+|[^\r\n\p{L}\p{P}\p{S}]?[\p{L}\p{M}]+
 *         | ?[\p{P}\p{S}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+ inside each
 *         piece, spans no alternative matches kept as pieces
 *       (pretok_classes_deepseek.v1.meta.json "patterns";
 *        crates/.../pretokenize/fast/deepseek_v3.rs:1-22), with the
 *        seven-class table O L M N PS WS CRLF of that meta file
 *       o200k (gpt-oss, o200k_base with contractions):
 *         [^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}]*[\p{Ll}\p{Lm}\p{Lo}\p{M}]+C?
 *         |[^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}]+[\p{Ll}\p{Lm}\p{Lo}\p{M}]*C?
 *         |\p{N}{1,K}| ?[^\s\p{L}\p{N}]+[\r\n/]*|\s*[\r\n]+|\s+(?!\S)|\s+
 *         with C = (?i:'s|'t|'re|'ve|'m|'ll|'d)
 *       (crates/.../pretokenize/options.rs O200k row; kernel_families.v1.json
 *        gpt_oss_120b: digits_max 3, contractions), with the seven-class
 *        table P U L C N S M (U = Lu Lt, L = Ll, C = Lm Lo; class table
 *        o200k_v4, whose sha256 the probed table reproduces); the o200k
 *        rows with contractions false drop C
 *       kimi (Kimi K3): [\p{Han}]+ first, then the o200k alternatives with
 *         the letter classes minus Han, \p{N}{1,3} (Han numbers too),
 *         ' ?[^\s\p{L}\p{N}]+[\r\n]*' (no '/' in the tail) and the
 *         whitespace ones (src/toktier/artifacts/conversion.py
 *         KIMI_PATTERN), with the ten-class table of kimi_v1 (the o200k
 *         seven without Han, HL HN HP; its sha256 the probed table
 *         reproduces)
 *     with \s / \p{L} / \p{N} membership read from the probed class table
 *     (classes P=0 L=1 N=2 S=3, pretok_kernel.cu:63) and the case folding
 *     of (?i:...) restricted to A-Z and U+017F (pretok_kernel.cu:153-158);
 *   - byte-level BPE with the HF `tokenizers` semantics the reference
 *     certifies against (pretok_kernel.cu:872-881): initial symbols are
 *     byte ids (bytes without an id are dropped, pretok_kernel.cu:1012-1021),
 *     then the adjacent pair of lowest merge rank is merged, leftmost
 *     first, until none is left; a min-heap of (rank, position) with stale
 *     entries skipped, which is the published HF algorithm
 *     (tokenizers 0.22.2, models/bpe/word.rs `merge_all`);
 *   - ignore_merges: a piece that is itself a vocabulary entry is emitted
 *     as that one token (pretok_kernel.cu:921-943, :1005-1008);
 *   - table lookups in the boundary format (src/toktier/kernels/
 *     bpe_tables.py:99-132: splitmix64 slot, linear probing, empty = ~0;
 *     FNV-1a-64 vocabulary keys with a byte recheck against the blob);
 *   - the NFC quick check (pretok_kernel.cu:2139-2181 and
 *     nfc_quick_check.v1.meta.json predicate).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "toktier_oracle.h"

enum { CP_ = 0, CL_ = 1, CN_ = 2, CS_ = 3 };

/* ------------------------------------------------------------ hashing */

static uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ULL;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
  return x ^ (x >> 31);
}

/* rank<<32|merged_id, or -1 */
static int64_t pair_lookup(const tko_tables* t, uint32_t l, uint32_t r) {
  uint64_t key = ((uint64_t)l << 32) | r;
  uint64_t mask = t->pair_count - 1;
  uint64_t i = splitmix64(key) & mask;
  for (;;) {
    uint64_t k = t->pair_keys[i];
    if (k == ~0ULL) return -1;
    if (k == key) return (int64_t)t->pair_vals[i];
    i = (i + 1) & mask;
  }
}

static int64_t vocab_lookup(const tko_tables* t, const uint8_t* s, int64_t m) {
  uint64_t h = 0xCBF29CE484222325ULL;
  for (int64_t j = 0; j < m; ++j) h = (h ^ s[j]) * 0x100000001B3ULL;
  uint64_t mask = t->vocab_count - 1;
  uint64_t i = splitmix64(h) & mask;
  for (;;) {
    uint64_t k = t->vocab_keys[i];
    if (k == ~0ULL) return -1;
    if (k == h) {
      uint64_t v = t->vocab_vals[i];
      int64_t len = (int64_t)((v >> 20) & 0x3FF);
      uint64_t off = v >> 30;
      if (len == m && memcmp(t->vocab_blob + off, s, (size_t)m) == 0)
        return (int64_t)(v & 0xFFFFF);
    }
    i = (i + 1) & mask;
  }
}

/* ------------------------------------------------------------- UTF-8 */

int64_t tko_utf8_decode(const uint8_t* s, int64_t nb, int32_t* cp,
                        int64_t* bo) {
  int64_t n = 0, i = 0;
  while (i < nb) {
    uint32_t b0 = s[i];
    int need;
    uint32_t v;
    if (b0 < 0x80) { need = 0; v = b0; }
    else if (b0 < 0xC0) return -1;
    else if (b0 < 0xE0) { need = 1; v = b0 & 0x1F; }
    else if (b0 < 0xF0) { need = 2; v = b0 & 0x0F; }
    else if (b0 < 0xF8) { need = 3; v = b0 & 0x07; }
    else return -1;
    for (int k = 1; k <= need; ++k) {
      if (i + k >= nb) return -1;
      uint32_t c = s[i + k];
      if ((c & 0xC0) != 0x80) return -1;
      v = (v << 6) | (c & 0x3F);
    }
    if ((need == 1 && v < 0x80) || (need == 2 && v < 0x800) ||
        (need == 3 && v < 0x10000) || v > 0x10FFFF ||
        (v >= 0xD800 && v <= 0xDFFF))
      return -1;
    if (cp) cp[n] = (int32_t)v;
    if (bo) bo[n] = i;
    ++n;
    i += need + 1;
  }
  return n;
}

/* -------------------------------------------------------- pretokenize */

static int fold(int32_t c) {
  if (c >= 'A' && c <= 'Z') return c + 32;
  if (c == 0x17F) return 's';
  return c;
}

static int is_crlf(int32_t c) { return c == '\r' || c == '\n'; }

/* End (exclusive, in chars) of the cl100k match that starts at char i. */
static int64_t match_cl100k(const int32_t* cp, const uint8_t* cl, int64_t i,
                            int64_t n, int K, int fold_case) {
  /* (?i:'s|'t|'re|'ve|'m|'ll|'d) -- first letters are distinct, so the
     alternatives cannot compete */
  if (cp[i] == '\'' && i + 1 < n) {
    int a = fold_case ? fold(cp[i + 1]) : cp[i + 1];
    if (a == 's' || a == 't' || a == 'm' || a == 'd') return i + 2;
    if (i + 2 < n) {
      int b = fold_case ? fold(cp[i + 2]) : cp[i + 2];
      if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') ||
          (a == 'l' && b == 'l'))
        return i + 3;
    }
  }
  /* [^\r\n\p{L}\p{N}]?\p{L}+ : the optional prefix first tries to take
     cp[i]; a letter is not in the prefix class, so then \p{L}+ starts at i */
  if (cl[i] == CL_) {
    int64_t j = i + 1;
    while (j < n && cl[j] == CL_) ++j;
    return j;
  }
  if (cl[i] != CN_ && !is_crlf(cp[i]) && i + 1 < n && cl[i + 1] == CL_) {
    int64_t j = i + 2;
    while (j < n && cl[j] == CL_) ++j;
    return j;
  }
  /* \p{N}{1,K} */
  if (cl[i] == CN_) {
    int64_t j = i + 1;
    while (j < n && cl[j] == CN_ && j - i < K) ++j;
    return j;
  }
  /*  ?[^\s\p{L}\p{N}]+[\r\n]* : with the space taken the run must start at
     i+1; without it cp[i] itself must be P */
  {
    int64_t j = -1;
    if (cp[i] == ' ') {
      if (i + 1 < n && cl[i + 1] == CP_) j = i + 1;
    } else if (cl[i] == CP_) {
      j = i;
    }
    if (j >= 0) {
      while (j < n && cl[j] == CP_) ++j;
      while (j < n && is_crlf(cp[j])) ++j;
      return j;
    }
  }
  /* the rest are whitespace alternatives: cp[i] is \s here */
  {
    int64_t e = i;
    while (e < n && cl[e] == CS_) ++e;
    /* \s*[\r\n]+ : \s* backs off until [\r\n]+ can start, i.e. the match
       ends right after the last CR/LF of the run */
    for (int64_t k = e - 1; k >= i; --k)
      if (is_crlf(cp[k])) return k + 1;
    /* \s+(?!\S) : the whole run at end of text, else one char shorter */
    if (e == n) return e;
    if (e - 1 > i) return e - 1;
    /* \s+ */
    return e;
  }
}

/* End of the r50k (GPT-2) match that starts at char i. */
static int64_t match_r50k(const int32_t* cp, const uint8_t* cl, int64_t i,
                          int64_t n) {
  if (cp[i] == '\'' && i + 1 < n) {
    int a = cp[i + 1];
    if (a == 's' || a == 't' || a == 'm' || a == 'd') return i + 2;
    if (i + 2 < n) {
      int b = cp[i + 2];
      if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') ||
          (a == 'l' && b == 'l'))
        return i + 3;
    }
  }
  /* ' ?\p{L}+', ' ?\p{N}+', ' ?[^\s\p{L}\p{N}]+' in that order */
  for (int want = CL_;; want = (want == CL_ ? CN_ : CP_)) {
    int64_t j = -1;
    if (cp[i] == ' ') {
      if (i + 1 < n && cl[i + 1] == want) j = i + 1;
    } else if (cl[i] == want) {
      j = i;
    }
    if (j >= 0) {
      while (j < n && cl[j] == want) ++j;
      return j;
    }
    if (want == CP_) break;
  }
  {
    int64_t e = i;
    while (e < n && cl[e] == CS_) ++e;
    if (e == n) return e;          /* \s+(?!\S) at end of text */
    if (e - 1 > i) return e - 1;   /* backed off by one */
    return e;                      /* \s+ */
  }
}

/* ---- DeepSeek: classes of pretok_classes_deepseek.v1.meta.json "enum" */
enum { DS_O = 0, DS_L = 1, DS_M = 2, DS_N = 3, DS_PS = 4, DS_WS = 5, DS_CR = 6 };

static int ds_cjk(int32_t c) {  /* the stage-2 class (meta "cjk_ranges") */
  return (c >= 0x4E00 && c <= 0x9FA5) || (c >= 0x3040 && c <= 0x30FF);
}
static int ascii_punct(int32_t c) {  /* meta "apunct" */
  return (c >= 0x21 && c <= 0x2F) || (c >= 0x3A && c <= 0x40) ||
         (c >= 0x5B && c <= 0x60) || (c >= 0x7B && c <= 0x7E);
}
static int ascii_alpha(int32_t c) {
  return (c >= 'A' && c <= 'Z') || (c >= 'a' && c <= 'z');
}
static int ds_lm(uint8_t k) { return k == DS_L || k == DS_M; }
static int ds_space(uint8_t k) { return k == DS_WS || k == DS_CR; }

/* End of the stage-3 match that starts at char i inside a piece ending at
 * n, or -1 when no alternative matches there. */
static int64_t match_deepseek(const int32_t* cp, const uint8_t* cl, int64_t i,
                              int64_t n) {
  const uint8_t k = cl[i];
  /* [ascii punct][A-Za-z]+ */
  if (ascii_punct(cp[i]) && i + 1 < n && ascii_alpha(cp[i + 1])) {
    int64_t j = i + 2;
    while (j < n && ascii_alpha(cp[j])) ++j;
    return j;
  }
  /* [^\r\n\p{L}\p{P}\p{S}]?[\p{L}\p{M}]+ : the optional class is O, M,
     N or non-CR/LF whitespace; it takes cp[i] when [\p{L}\p{M}]+ can
     follow, else the run has to start at i */
  if (k != DS_L && k != DS_PS && k != DS_CR && i + 1 < n && ds_lm(cl[i + 1])) {
    int64_t j = i + 2;
    while (j < n && ds_lm(cl[j])) ++j;
    return j;
  }
  if (ds_lm(k)) {
    int64_t j = i + 1;
    while (j < n && ds_lm(cl[j])) ++j;
    return j;
  }
  /*  ?[\p{P}\p{S}]+[\r\n]* */
  {
    int64_t j = -1;
    if (cp[i] == ' ') {
      if (i + 1 < n && cl[i + 1] == DS_PS) j = i + 1;
    } else if (k == DS_PS) {
      j = i;
    }
    if (j >= 0) {
      while (j < n && cl[j] == DS_PS) ++j;
      while (j < n && cl[j] == DS_CR) ++j;
      return j;
    }
  }
  if (!ds_space(k)) return -1;
  {
    int64_t e = i;
    while (e < n && ds_space(cl[e])) ++e;
    /* \s*[\r\n]+ ends right after the run's last CR/LF */
    for (int64_t q = e - 1; q >= i; --q)
      if (cl[q] == DS_CR) return q + 1;
    if (e == n) return e;         /* \s+(?!\S) at the end of the piece */
    if (e - 1 > i) return e - 1;  /* backed off by one */
    return e;                     /* \s+ */
  }
}

/* The three stages over chars [0, n): stage 1 cuts \p{N}{1,K} groups
 * (leftmost, so a run splits into K-char groups from its start) and keeps
 * the text between them; stage 2 cuts each such text into CJK runs and the
 * rest; stage 3 runs the main pattern inside each of those, and a span no
 * alternative matches at (a run of O chars not followed by a letter or
 * mark) stays one piece. */
static int64_t pieces_deepseek(const int32_t* cp, const uint8_t* cl,
                               const int64_t* bo, int64_t n, int K,
                               int64_t* starts) {
  int64_t p = 0, i = 0;
  while (i < n) {
    if (cl[i] == DS_N) {
      starts[p++] = bo[i];
      int64_t j = i + 1;
      while (j < n && cl[j] == DS_N && j - i < K) ++j;
      i = j;
      continue;
    }
    const int c = ds_cjk(cp[i]);
    int64_t end = i + 1;
    while (end < n && cl[end] != DS_N && ds_cjk(cp[end]) == c) ++end;
    int gap = 0;
    while (i < end) {
      const int64_t m = match_deepseek(cp, cl, i, end);
      if (m < 0) {
        if (!gap) starts[p++] = bo[i];
        gap = 1;
        ++i;
      } else {
        starts[p++] = bo[i];
        gap = 0;
        i = m;
      }
    }
  }
  return p;
}

/* ---- o200k: classes P U L C N S M (o200k_v4); kimi adds HL HN HP
 * (kimi_v1: Han letters, Han numbers, other Han), and its letter classes
 * hold no Han */
enum { OK_P = 0, OK_U = 1, OK_L = 2, OK_C = 3, OK_N = 4, OK_S = 5, OK_M = 6,
       OK_HL = 7, OK_HN = 8, OK_HP = 9 };

static int ok_a(uint8_t k) { return k == OK_U || k == OK_C || k == OK_M; }
static int ok_b(uint8_t k) { return k == OK_L || k == OK_C || k == OK_M; }
static int ok_han(uint8_t k) { return k >= OK_HL; }
/* [^\r\n\p{L}\p{N}] (kimi: Han that is neither letter nor number too) */
static int ok_q(uint8_t k, int32_t c) {
  return (k == OK_P || k == OK_M || k == OK_S || k == OK_HP) && !is_crlf(c);
}
/* [^\s\p{L}\p{N}] */
static int ok_pm(uint8_t k) { return k == OK_P || k == OK_M || k == OK_HP; }

/* [A]*[B]+ from t (A = Lu Lt Lm Lo M, B = Ll Lm Lo M): A* takes the
 * longest run, then gives characters back until B+ can start; B+ then runs
 * to the end of the B characters. End, or -1. */
static int64_t ok_letters1(const uint8_t* cl, int64_t t, int64_t n) {
  int64_t a = t;
  while (a < n && ok_a(cl[a])) ++a;
  if (a < n && cl[a] == OK_L) {
    int64_t b = a + 1;
    while (b < n && ok_b(cl[b])) ++b;
    return b;
  }
  /* backing off: the last character of the run that B+ accepts (C or M);
     the one after it is U or ends the run, so B+ takes just it */
  for (int64_t j = a - 1; j >= t; --j)
    if (ok_b(cl[j])) return j + 1;
  return -1;
}

/* [A]+[B]* from t. */
static int64_t ok_letters2(const uint8_t* cl, int64_t t, int64_t n) {
  int64_t a = t;
  while (a < n && ok_a(cl[a])) ++a;
  if (a == t) return -1;
  while (a < n && ok_b(cl[a])) ++a;
  return a;
}

/* (?i:'s|'t|'re|'ve|'m|'ll|'d)? after a letter match ending at e */
static int64_t ok_contraction(const int32_t* cp, int64_t e, int64_t n) {
  if (e + 1 < n && cp[e] == '\'') {
    int a = fold(cp[e + 1]);
    if (a == 's' || a == 't' || a == 'm' || a == 'd') return e + 2;
    if (e + 2 < n) {
      int b = fold(cp[e + 2]);
      if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') ||
          (a == 'l' && b == 'l'))
        return e + 3;
    }
  }
  return e;
}

/* End of the o200k / kimi match that starts at char i. kimi: [\p{Han}]+
 * first, \p{N} and [^\s\p{L}\p{N}] take the Han numbers and the other Han,
 * and the punctuation tail is [\r\n]* (o200k: [\r\n/]*). Each letter
 * alternative is tried with the optional prefix first taking cp[i], then
 * without it; `contr` false drops the contraction suffix. */
static int64_t match_o200k(const int32_t* cp, const uint8_t* cl, int64_t i,
                           int64_t n, int K, int kimi, int contr) {
  if (kimi && ok_han(cl[i])) {
    int64_t j = i + 1;
    while (j < n && ok_han(cl[j])) ++j;
    return j;
  }
  const int q = ok_q(cl[i], cp[i]);
  int64_t e = -1;
  if (q && i + 1 < n) e = ok_letters1(cl, i + 1, n);
  if (e < 0) e = ok_letters1(cl, i, n);
  if (e < 0 && q && i + 1 < n) e = ok_letters2(cl, i + 1, n);
  if (e < 0) e = ok_letters2(cl, i, n);
  if (e >= 0) return contr ? ok_contraction(cp, e, n) : e;
  if (cl[i] == OK_N || cl[i] == OK_HN) {
    int64_t j = i + 1;
    while (j < n && (cl[j] == OK_N || cl[j] == OK_HN) && j - i < K) ++j;
    return j;
  }
  /*  ?[^\s\p{L}\p{N}]+[\r\n/]* (kimi: [\r\n]*) */
  {
    int64_t j = -1;
    if (cp[i] == ' ') {
      if (i + 1 < n && ok_pm(cl[i + 1])) j = i + 1;
    } else if (ok_pm(cl[i])) {
      j = i;
    }
    if (j >= 0) {
      while (j < n && ok_pm(cl[j])) ++j;
      while (j < n && (is_crlf(cp[j]) || (!kimi && cp[j] == '/'))) ++j;
      return j;
    }
  }
  {
    int64_t e2 = i;
    while (e2 < n && cl[e2] == OK_S) ++e2;
    for (int64_t k = e2 - 1; k >= i; --k)
      if (is_crlf(cp[k])) return k + 1;
    if (e2 == n) return e2;
    if (e2 - 1 > i) return e2 - 1;
    return e2;
  }
}

/* Laguna's stage 0, (?:\r?\n)+ split MergedWithNext
 * (src/toktier/kernels/pretok_kernel.cu:76-86): the first position after
 * i where a match of the pattern starts, or n. Scanning left to right, a
 * match starts at a '\n' or at a '\r' followed by '\n', and then takes
 * every (\r?\n) unit that follows it. */
static int64_t next_newline_run(const int32_t* cp, int64_t i, int64_t n) {
  int64_t q = i;
  /* if the part starts inside a match (the match opened it), skip it */
  while (q < n) {
    if (cp[q] == '\n') { ++q; continue; }
    if (cp[q] == '\r' && q + 1 < n && cp[q + 1] == '\n') { q += 2; continue; }
    break;
  }
  for (; q < n; ++q) {
    if (cp[q] == '\n') return q;
    if (cp[q] == '\r' && q + 1 < n && cp[q + 1] == '\n') return q;
  }
  return n;
}

int64_t tko_pretokenize(const tko_tables* t, const uint8_t* s, int64_t nb,
                        int64_t* starts) {
  int32_t* cp = (int32_t*)malloc(sizeof(int32_t) * (size_t)(nb + 1));
  int64_t* bo = (int64_t*)malloc(sizeof(int64_t) * (size_t)(nb + 1));
  uint8_t* cl = (uint8_t*)malloc((size_t)(nb + 1));
  if (!cp || !bo || !cl) { free(cp); free(bo); free(cl); return -2; }
  int64_t n = tko_utf8_decode(s, nb, cp, bo);
  if (n < 0) { free(cp); free(bo); free(cl); return -1; }
  for (int64_t i = 0; i < n; ++i) cl[i] = t->cls[cp[i]];
  int64_t p = 0, i = 0;
  if (t->ruleset == TKO_RULESET_DEEPSEEK) i = n;
  if (t->ruleset == TKO_RULESET_DEEPSEEK)
    p = pieces_deepseek(cp, cl, bo, n, t->digits_max, starts);
  while (i < n) {
    /* the part the regex runs in: the whole text, or (Laguna) up to the
       next start of a (?:\r?\n)+ match, since that stage splits with
       behavior MergedWithNext: each newline run opens a new part */
    int64_t end = n;
    if (t->ruleset == TKO_RULESET_LAGUNA) end = next_newline_run(cp, i, n);
    while (i < end) {
      starts[p++] = bo[i];
      const int64_t j = t->ruleset == TKO_RULESET_R50K
              ? match_r50k(cp, cl, i, end)
              : t->ruleset == TKO_RULESET_O200K || t->ruleset == TKO_RULESET_KIMI
              ? match_o200k(cp, cl, i, end, t->digits_max,
                            t->ruleset == TKO_RULESET_KIMI, t->contractions)
              : match_cl100k(cp, cl, i, end, t->digits_max, 1);
      if (j <= i) {  /* a class the ruleset does not know: no match */
        free(cp); free(bo); free(cl);
        return TKO_E_CLASS;
      }
      i = j;
    }
  }
  starts[p] = nb;
  free(cp); free(bo); free(cl);
  return p;
}

/* ---------------------------------------------------------------- BPE */

typedef struct { uint32_t rank; int32_t pos; } hent;

static int hless(hent a, hent b) {
  return a.rank < b.rank || (a.rank == b.rank && a.pos < b.pos);
}

static void hpush(hent* h, int64_t* n, hent e) {
  int64_t i = (*n)++;
  h[i] = e;
  while (i > 0) {
    int64_t p = (i - 1) / 2;
    if (!hless(h[i], h[p])) break;
    hent tmp = h[i]; h[i] = h[p]; h[p] = tmp;
    i = p;
  }
}

static hent hpop(hent* h, int64_t* n) {
  hent top = h[0];
  h[0] = h[--(*n)];
  int64_t i = 0;
  for (;;) {
    int64_t l = 2 * i + 1, r = l + 1, m = i;
    if (l < *n && hless(h[l], h[m])) m = l;
    if (r < *n && hless(h[r], h[m])) m = r;
    if (m == i) break;
    hent tmp = h[i]; h[i] = h[m]; h[m] = tmp;
    i = m;
  }
  return top;
}

int64_t tko_bpe(const tko_tables* t, const uint8_t* s, int64_t m,
                uint32_t* out) {
  if (m <= 0) return 0;
  if (t->ignore_merges) {
    int64_t hit = vocab_lookup(t, s, m);
    if (hit >= 0) { out[0] = (uint32_t)hit; return 1; }
  }
  int32_t* id = (int32_t*)malloc(sizeof(int32_t) * (size_t)m);
  int32_t* nx = (int32_t*)malloc(sizeof(int32_t) * (size_t)m);
  int32_t* pv = (int32_t*)malloc(sizeof(int32_t) * (size_t)m);
  hent* heap = (hent*)malloc(sizeof(hent) * (size_t)(3 * m + 4));
  if (!id || !nx || !pv || !heap) {
    free(id); free(nx); free(pv); free(heap);
    return -2;
  }
  int32_t k = 0;
  for (int64_t j = 0; j < m; ++j) {
    int32_t v = t->byte_id[s[j]];
    if (v >= 0) id[k++] = v;  /* bytes without an id are dropped */
  }
  for (int32_t j = 0; j < k; ++j) { nx[j] = j + 1 < k ? j + 1 : -1; pv[j] = j - 1; }
  int64_t hn = 0;
  for (int32_t j = 0; j + 1 < k; ++j) {
    int64_t v = pair_lookup(t, (uint32_t)id[j], (uint32_t)id[j + 1]);
    if (v >= 0) hpush(heap, &hn, (hent){(uint32_t)(v >> 32), j});
  }
  while (hn > 0) {
    hent e = hpop(heap, &hn);
    int32_t j = e.pos;
    if (id[j] < 0 || nx[j] < 0) continue;          /* dead or last */
    int32_t r = nx[j];
    int64_t v = pair_lookup(t, (uint32_t)id[j], (uint32_t)id[r]);
    if (v < 0 || (uint32_t)(v >> 32) != e.rank) continue;   /* stale */
    id[j] = (int32_t)(v & 0xFFFFFFFF);
    id[r] = -1;
    nx[j] = nx[r];
    if (nx[j] >= 0) pv[nx[j]] = j;
    if (pv[j] >= 0) {
      int64_t w = pair_lookup(t, (uint32_t)id[pv[j]], (uint32_t)id[j]);
      if (w >= 0) hpush(heap, &hn, (hent){(uint32_t)(w >> 32), pv[j]});
    }
    if (nx[j] >= 0) {
      int64_t w = pair_lookup(t, (uint32_t)id[j], (uint32_t)id[nx[j]]);
      if (w >= 0) hpush(heap, &hn, (hent){(uint32_t)(w >> 32), j});
    }
  }
  int64_t c = 0;
  for (int32_t j = (k > 0 ? 0 : -1); j >= 0; j = nx[j]) out[c++] = (uint32_t)id[j];
  free(id); free(nx); free(pv); free(heap);
  return c;
}

/* ---------------------------------------------------------------- NFC */

int tko_nfc_qc(const tko_tables* t, const uint8_t* s, int64_t nb) {
  int32_t* cp = (int32_t*)malloc(sizeof(int32_t) * (size_t)(nb + 1));
  if (!cp) return -2;
  int64_t n = tko_utf8_decode(s, nb, cp, NULL);
  if (n < 0) { free(cp); return -1; }
  int ok = 1;
  uint8_t prev = 0;
  for (int64_t i = 0; i < n && ok; ++i) {
    uint8_t v = t->nfc_qc[cp[i]];
    if (v == 255 || (i > 0 && prev > v && v != 0)) ok = 0;
    prev = v;
  }
  free(cp);
  return ok;
}

/* ------------------------------------------------------------- encode */

int64_t tko_encode(const tko_tables* t, const uint8_t* s, int64_t nb,
                   uint32_t* out, int64_t cap) {
  if (nb == 0) return 0;
  if (t->needs_nfc && t->nfc_qc) {
    int q = tko_nfc_qc(t, s, nb);
    if (q < 0) return q == -1 ? TKO_E_UTF8 : TKO_E_NOMEM;
    if (q == 0) return TKO_E_NEEDS_NFC;
  }
  int64_t* starts = (int64_t*)malloc(sizeof(int64_t) * (size_t)(nb + 1));
  if (!starts) return TKO_E_NOMEM;
  int64_t p = tko_pretokenize(t, s, nb, starts);
  if (p < 0) { free(starts); return p == -1 ? TKO_E_UTF8 : TKO_E_NOMEM; }
  int64_t total = 0;
  for (int64_t k = 0; k < p; ++k) {
    int64_t a = starts[k], b = starts[k + 1];
    if (total + (b - a) > cap) { free(starts); return TKO_E_CAP; }
    int64_t c = tko_bpe(t, s + a, b - a, out + total);
    if (c < 0) { free(starts); return TKO_E_NOMEM; }
    total += c;
  }
  free(starts);
  return total;
}

/* ------------------------------------------------- added-token split */

/* HF tokenizers 0.22.2 splits the text at its added-token literals before
 * normalization and pretokenization (the added vocabulary's Aho-Corasick
 * search in leftmost-longest mode; the reference calls the same split,
 * src/toktier/frontend/added.py:490-533, and joins the parts,
 * :544-555): scanning left to right, the first position where a literal
 * matches takes the longest literal matching there, and the scan resumes
 * after it. Each literal is its own id; the text between two literals is
 * encoded as a text of its own (its own quick check, pretokenization and
 * merges). Literals here carry no single_word / lstrip / rstrip flag. */
int64_t tko_encode_added(const tko_tables* t, const tko_added* a,
                         const uint8_t* s, int64_t nb, uint32_t* out,
                         int64_t cap) {
  uint8_t first[256];
  memset(first, 0, sizeof first);
  for (int64_t k = 0; k < a->n; ++k)
    if (a->offsets[k + 1] > a->offsets[k]) first[a->blob[a->offsets[k]]] = 1;
  int64_t total = 0, seg = 0, i = 0;
  while (i <= nb) {
    int64_t best = -1, blen = 0;
    if (i < nb && first[s[i]]) {
      for (int64_t k = 0; k < a->n; ++k) {
        const int64_t L = (int64_t)(a->offsets[k + 1] - a->offsets[k]);
        if (L > blen && L <= nb - i &&
            memcmp(s + i, a->blob + a->offsets[k], (size_t)L) == 0) {
          best = k;
          blen = L;
        }
      }
    }
    if (best >= 0 || i == nb) {
      if (i > seg) {
        int64_t c = tko_encode(t, s + seg, i - seg, out + total, cap - total);
        if (c < 0) return c;
        total += c;
      }
      if (i == nb) break;
      if (total + 1 > cap) return TKO_E_CAP;
      out[total++] = a->ids[best];
      i += blen;
      seg = i;
    } else {
      ++i;
    }
  }
  return total;
}
