"""Family descriptions for the GPU fresh-encode path.

A family fixes everything that changes token ids on this path: the split
regex (and with it the device ruleset), the digit group width, whether the
model ignores merges for whole-vocabulary pieces, and whether the
artifact declares an NFC normalizer.

Reference data this mirrors:
- ``src/toktier/kernels/tables/kernel_families.v1.json:103-117``
  (``qwen3_8b``: ruleset cl100k, digits_max 1, contractions; ``llama_3_1_8b``:
  digits_max 3).
- Split patterns: ``crates/toktier-gigatoken-core/src/pretokenize/options.rs:118-132``
  (GPT2, Qwen2, Olmo3/Llama-3 rows).
- ``NativePrebuiltGpuConfig`` fields ``ruleset``, ``digits_max``,
  ``contractions``, ``needs_nfc``, ``ignore_merges``
  (``crates/toktier-routing-core/src/gpu.rs:22-38``).

DeepSeek V3 (``kernel_families.v1.json`` family ``deepseek_v3``: band and
ruleset deepseek, class table deepseek_v1, contractions false, digits_max
3 from ``pretok_classes_deepseek.v1.meta.json``) splits in three stages
(that meta file's ``patterns``); its device ruleset is ``deepseek``.

GPT-2 is not a GPU family in the reference (its r50k split exists only in
the CPU scanner ``crates/toktier-gigatoken-core/src/pretokenize/fast/r50k.rs``);
here it gets its own device ruleset, ``r50k``.
"""

from __future__ import annotations

from dataclasses import dataclass

__all__ = ["Family", "FAMILIES", "family", "class_table_name",
           "RULESET_CL100K", "RULESET_R50K",
           "RULESET_LAGUNA", "RULESET_DEEPSEEK", "RULESET_O200K",
           "RULESET_KIMI", "DEEPSEEK_STAGES", "O200K_PATTERN", "KIMI_PATTERN",
           "QWEN35_PATTERN", "NEMOTRON_PATTERN"]

#: Device ruleset ids (the ``ruleset`` field of the engine config).
RULESET_CL100K = 0
RULESET_R50K = 1
#: Laguna-S-2.1's two-stage Split group: a newline-run split that keeps each
#: run with the text after it, then the Qwen2 pattern inside each part
#: (``src/toktier/kernels/pretok_kernel.cu:76-86``;
#: ``kernel_families.v1.json`` family ``laguna_s_2_1``: band cl100k,
#: ruleset laguna, digits_max 1, class table cl100k_v3).
RULESET_LAGUNA = 2

#: DeepSeek V3 / V4: three Split(Isolated) stages, applied in order
#: (``pretok_classes_deepseek.v1.meta.json`` ``patterns``).
RULESET_DEEPSEEK = 3

#: o200k (gpt-oss; ``kernel_families.v1.json`` family ``gpt_oss_120b``:
#: band and ruleset o200k, class table o200k_v4, digits_max 3,
#: contractions true): letters split by case, contraction suffixes,
#: digit groups of three.
RULESET_O200K = 4

#: kimi (``kernel_families.v1.json`` family ``kimi_k3``: band and ruleset
#: kimi, class table kimi_v1, digits_max 3, contractions true): o200k with
#: a leading [\p{Han}]+ branch, letter classes without Han, and a
#: punctuation tail without '/'.
RULESET_KIMI = 5

#: The Kimi pre-tokenizer pattern (``src/toktier/artifacts/conversion.py``
#: KIMI_PATTERN; sha256 de5781783b19... as pretok_classes_kimi.v1.meta.json
#: ``pattern_sha256``).
KIMI_PATTERN = "|".join((
    r"[\p{Han}]+",
    r"[^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}&&[^\p{Han}]]*"
    r"[\p{Ll}\p{Lm}\p{Lo}\p{M}&&[^\p{Han}]]+(?i:'s|'t|'re|'ve|'m|'ll|'d)?",
    r"[^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}&&[^\p{Han}]]+"
    r"[\p{Ll}\p{Lm}\p{Lo}\p{M}&&[^\p{Han}]]*(?i:'s|'t|'re|'ve|'m|'ll|'d)?",
    r"\p{N}{1,3}",
    r" ?[^\s\p{L}\p{N}]+[\r\n]*",
    r"\s*[\r\n]+",
    r"\s+(?!\S)",
    r"\s+",
))

#: Laguna's stage 0, split with behavior MergedWithNext.
LAGUNA_STAGE0 = r"(?:\r?\n)+"

QWEN2_PATTERN = (
    r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}"
    r"| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+"
)
LLAMA3_PATTERN = (
    r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}{1,3}"
    r"| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+"
)
DEEPSEEK_STAGES = (
    r"\p{N}{1,3}",
    "[\u4e00-\u9fa5\u3040-\u309f\u30a0-\u30ff]+",
    # (CR and LF are literal characters in the artifact's pattern)
    "[!\"#$%&'()*+,\\-./:;<=>?@\\[\\\\\\]^_`{|}~][A-Za-z]+"
    "|[^\r\n\\p{L}\\p{P}\\p{S}]?[\\p{L}\\p{M}]+| ?[\\p{P}\\p{S}]+[\r\n]*"
    "|\\s*[\r\n]+|\\s+(?!\\S)|\\s+",
)

#: o200k_base with contractions (gpt-oss; ``options.rs`` O200k row; the
#: oracle's and the device's ruleset 4).
O200K_PATTERN = (
    r"[^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}]*[\p{Ll}\p{Lm}\p{Lo}\p{M}]+"
    r"(?i:'s|'t|'re|'ve|'m|'ll|'d)?"
    r"|[^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}]+[\p{Ll}\p{Lm}\p{Lo}\p{M}]*"
    r"(?i:'s|'t|'re|'ve|'m|'ll|'d)?"
    r"|\p{N}{1,3}| ?[^\s\p{L}\p{N}]+[\r\n/]*|\s*[\r\n]+|\s+(?!\S)|\s+"
)

#: Qwen3.5 (``options.rs`` Qwen35 row): the Qwen2 pattern with marks in
#: the letter run and out of the punctuation run; the cl100k ruleset over
#: the marks-as-letters class table (``kernel_families.v1.json`` family
#: ``qwen3_5_08b``: class table cl100k_m2l_v3, digits_max 1).
QWEN35_PATTERN = (
    r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?[\p{L}\p{M}]+|\p{N}"
    r"| ?[^\s\p{L}\p{M}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+"
)

#: Nemotron-3 (``options.rs`` Nemotron row; ``pretokenize/fast/nemotron.rs``):
#: o200k without the contraction suffix and with single-digit groups
#: (``kernel_families.v1.json`` families ``nemotron_3_nano_4b`` and
#: ``ministral_3_8b``: ruleset o200k, digits_max 1, contractions false).
NEMOTRON_PATTERN = (
    r"[^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}]*[\p{Ll}\p{Lm}\p{Lo}\p{M}]+"
    r"|[^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}]+[\p{Ll}\p{Lm}\p{Lo}\p{M}]*"
    r"|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n/]*|\s*[\r\n]+|\s+(?!\S)|\s+"
)

#: The pattern HF ``ByteLevel(use_regex=True)`` applies (GPT-2).
GPT2_PATTERN = (
    r"'s|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+"
    r"|\s+(?!\S)|\s+"
)


@dataclass(frozen=True)
class Family:
    name: str
    ruleset: int           # RULESET_CL100K / _R50K / _LAGUNA / _DEEPSEEK / _O200K / _KIMI
    ruleset_name: str      # "cl100k" / "r50k" / "laguna" / "deepseek" / "o200k" / "kimi"
    pattern: str
    digits_max: int        # digit group width (cl100k); 0 = unbounded (r50k)
    contractions_fold: bool  # (?i:...) contractions (cl100k) vs case-sensitive
    needs_nfc: bool
    ignore_merges: bool
    vocab_size: int        # regular (model) vocabulary size of the real artifact
    hf_repo: str           # where the real artifact lives (not fetched here)
    real_sha256: str | None  # pinned sha256 of the real tokenizer.json, if any
    # (o200k) the contraction suffix is part of the letter alternatives
    contractions: bool = True
    # the class table the ruleset reads (kernel_families.v1.json names);
    # "" for the ruleset's default
    class_table: str = ""


FAMILIES: dict[str, Family] = {
    "qwen3_8b": Family(
        name="qwen3_8b", ruleset=RULESET_CL100K, ruleset_name="cl100k",
        pattern=QWEN2_PATTERN, digits_max=1, contractions_fold=True,
        needs_nfc=True, ignore_merges=False, vocab_size=151643,
        hf_repo="Qwen/Qwen3-8B",
        # src/toktier/artifacts/tables/artifact_manifest.v1.json pin (11,422,654 B)
        real_sha256="aeb13307a71acd8fe81861d94ad54ab689df773318809eed3cbe794b4492dae4",
    ),
    "llama_3_1_8b": Family(
        name="llama_3_1_8b", ruleset=RULESET_CL100K, ruleset_name="cl100k",
        pattern=LLAMA3_PATTERN, digits_max=3, contractions_fold=True,
        needs_nfc=False, ignore_merges=True, vocab_size=128000,
        hf_repo="meta-llama/Llama-3.1-8B",
        # same manifest (9,085,658 B)
        real_sha256="76e48799b099d43365bd24ccd8ecc5aedac831718da780552f03b0a6eb4412aa",
    ),
    "laguna_s_2_1": Family(
        name="laguna_s_2_1", ruleset=RULESET_LAGUNA, ruleset_name="laguna",
        pattern=QWEN2_PATTERN, digits_max=1, contractions_fold=True,
        # the stand-in declares no normalizer; the engine takes either
        needs_nfc=False, ignore_merges=False,
        # vocabulary size of the stand-in (the real artifact's is not
        # recorded in the reference)
        vocab_size=100000,
        hf_repo="poolside/Laguna-S-2.1",
        # src/toktier/artifacts/tables/artifact_manifest.v1.json pin (7,287,677 B)
        real_sha256="809240f7a182cde859a4fc4ebc902e619a173d507e99304c1092aa04e7a6658e",
    ),
    "deepseek_v3": Family(
        name="deepseek_v3", ruleset=RULESET_DEEPSEEK, ruleset_name="deepseek",
        pattern=DEEPSEEK_STAGES[2], digits_max=3, contractions_fold=False,
        # the artifact declares an empty normalizer sequence
        needs_nfc=False, ignore_merges=False, vocab_size=128000,
        hf_repo="deepseek-ai/DeepSeek-V3",
        # src/toktier/artifacts/tables/artifact_manifest.v1.json pin (7,847,652 B)
        real_sha256="621ac2e32d0dba658404412318818aaa8ce8cda492e59830109d8da6b517fb41",
    ),
    "gpt_oss_120b": Family(
        name="gpt_oss_120b", ruleset=RULESET_O200K, ruleset_name="o200k",
        pattern=O200K_PATTERN, digits_max=3, contractions_fold=True,
        # tiktoken-derived, as Llama-3: no normalizer, whole-vocabulary
        # pieces first
        needs_nfc=False, ignore_merges=True, vocab_size=199998,
        hf_repo="openai/gpt-oss-120b",
        # src/toktier/artifacts/tables/artifact_manifest.v1.json pin (27,868,174 B)
        real_sha256="0614fe83cadab421296e664e1f48f4261fa8fef6e03e63bb75c20f38e37d07d3",
    ),
    "kimi_k3": Family(
        name="kimi_k3", ruleset=RULESET_KIMI, ruleset_name="kimi",
        pattern=KIMI_PATTERN, digits_max=3, contractions_fold=True,
        # converted from tiktoken ranks (artifact_conversions.v1.json
        # kimi_tiktoken_v1): no normalizer, whole-vocabulary pieces first
        needs_nfc=False, ignore_merges=True, vocab_size=163584,
        hf_repo="moonshotai/Kimi-K3",
        # src/toktier/artifacts/tables/artifact_manifest.v1.json pin (9,703,692 B)
        real_sha256="773c2476259d9e092bba48d1f4840aaf584fa87cd5083a7e33b54d6d6f9feb77",
    ),
    "qwen3_5_08b": Family(
        name="qwen3_5_08b", ruleset=RULESET_CL100K, ruleset_name="cl100k",
        pattern=QWEN35_PATTERN, digits_max=1, contractions_fold=True,
        needs_nfc=True, ignore_merges=False,
        # vocabulary size of the stand-in (the real artifact's is not
        # recorded in the reference)
        vocab_size=151643,
        hf_repo="Qwen/Qwen3.5-0.8B",
        # src/toktier/artifacts/tables/artifact_manifest.v1.json pin (12,807,982 B)
        real_sha256="5f9e4d4901a92b997e463c1f46055088b6cca5ca61a6522d1b9f64c4bb81cb42",
        class_table="cl100k_m2l_v3",
    ),
    "nemotron_3_nano_4b": Family(
        name="nemotron_3_nano_4b", ruleset=RULESET_O200K, ruleset_name="o200k",
        pattern=NEMOTRON_PATTERN, digits_max=1, contractions_fold=False,
        # tiktoken-derived vocabulary, as gpt-oss: no normalizer,
        # whole-vocabulary pieces first
        needs_nfc=False, ignore_merges=True,
        # vocabulary size of the stand-in (the real artifact's is not
        # recorded in the reference)
        vocab_size=131072,
        hf_repo="nvidia/NVIDIA-Nemotron-3-Nano-4B-BF16",
        # src/toktier/artifacts/tables/artifact_manifest.v1.json pin (17,077,484 B)
        real_sha256="623c34567aebb18582765289fbe23d901c62704d6518d71866e0e58db892b5b7",
        contractions=False,
    ),
    "gpt2": Family(
        name="gpt2", ruleset=RULESET_R50K, ruleset_name="r50k",
        pattern=GPT2_PATTERN, digits_max=0, contractions_fold=False,
        needs_nfc=False, ignore_merges=False, vocab_size=50257,
        hf_repo="openai-community/gpt2", real_sha256=None,
    ),
}


def class_table_name(fam: Family) -> str:
    """The reference name of the class table the family's ruleset reads."""
    if fam.class_table:
        return fam.class_table
    return {"deepseek": "deepseek_v1", "o200k": "o200k_v4",
            "kimi": "kimi_v1"}.get(fam.ruleset_name, "cl100k_v3")


def family(name: str) -> Family:
    try:
        return FAMILIES[name]
    except KeyError:
        raise KeyError(
            f"unknown family {name!r}; known: {sorted(FAMILIES)}"
        ) from None
