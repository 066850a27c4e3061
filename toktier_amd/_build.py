"""Build ``libtoktier_hip.so`` for gfx950 with hipcc (in-tree).

The library holds the device code object (gfx950) and the C-ABI host
engine. A manifest beside it records the sha256 of the library, the
offload architecture, the hipcc version and the exported ``tk_*`` symbols
(the role of the reference's ``tools/build_fatbin.py`` manifest).
"""

from __future__ import annotations

import hashlib
import json
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
ABI_HEADER = ROOT / "include" / "toktier_hip.h"
LIBDIR = PKG / "_lib"
LIB = LIBDIR / "libtoktier_hip.so"
MANIFEST = LIBDIR / "manifest.json"
ARCH = "gfx950"

SOURCES = ["tk_device.hip", "tk_added.hip", "tk_engine.cpp"]


def hashed_files() -> dict[str, Path]:
    """Every file the code object depends on, by the name the manifest
    records: all of ``csrc/`` (the compiled sources and the headers they
    include) and the C-ABI header."""
    files = {f"csrc/{f.name}": f for f in sorted(CSRC.iterdir())
             if f.is_file() and f.suffix in (".hip", ".cpp", ".h")}
    files["include/toktier_hip.h"] = ABI_HEADER
    return files


def source_digests() -> dict[str, str]:
    return {name: hashlib.sha256(f.read_bytes()).hexdigest()
            for name, f in hashed_files().items()}


def library_digest(lib: Path | None = None) -> str:
    lib = LIB if lib is None else lib
    return hashlib.sha256(b"toktier-hip-lib\0" + lib.read_bytes()).hexdigest()


HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Wall", "-Wno-unused-function",
    # packed FP32 instructions stay off on this pool (no float code here)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or Path(cand).exists()):
            return cand
    return "hipcc"


def exported_symbols(lib: Path) -> list[str]:
    nm = "/opt/rocm/llvm/bin/llvm-nm"
    if not Path(nm).exists():
        nm = "nm"
    out = subprocess.run([nm, "-D", "--defined-only", str(lib)],
                         capture_output=True, text=True, check=True).stdout
    return sorted({line.split()[-1] for line in out.splitlines()
                   if line.split() and line.split()[-1].startswith("tk_")})


def build_key(sources: dict, flags: list, hipcc: list) -> str:
    """Digest of what determines the code object: the sources, the flags
    and the compiler version. hipcc gives each compile a random unit id,
    so two builds of the same sources differ in a few bytes of the library
    and its own sha256 cannot name a build across rebuilds; this key can
    (the committed counter summaries are matched on it)."""
    body = json.dumps({"sources": sources, "flags": flags, "hipcc": hipcc,
                       "arch": ARCH}, sort_keys=True)
    return hashlib.sha256(b"toktier-hip-build\0" + body.encode()).hexdigest()


def build(verbose: bool = False) -> Path:
    LIBDIR.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(f".so.tmp{os.getpid()}")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-o", str(tmp),
           *[str(CSRC / s) for s in SOURCES]]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc build of libtoktier_hip.so failed")
    os.replace(tmp, LIB)
    ver = subprocess.run([_hipcc(), "--version"], capture_output=True,
                         text=True).stdout.strip().splitlines()
    digest = library_digest()
    sources = source_digests()
    MANIFEST.write_text(json.dumps({
        "library": LIB.name,
        "sha256_domain": "toktier-hip-lib",
        "sha256": digest,
        "build_key": build_key(sources, HIPCC_FLAGS, ver[:2]),
        "architecture": ARCH,
        "hipcc": ver[:2],
        "flags": HIPCC_FLAGS,
        "sources": sources,
        "symbols": exported_symbols(LIB),
    }, indent=1) + "\n")
    return LIB


def verify(manifest: dict | None = None) -> str | None:
    """None when the library on disk is the one the manifest describes and
    the sources it was built from are unchanged; else what differs (a
    stale library, or sources edited after the build)."""
    try:
        m = manifest if manifest is not None else json.loads(MANIFEST.read_text())
    except (OSError, ValueError) as err:
        return f"manifest unreadable: {err}"
    if not LIB.exists():
        return "library missing"
    if library_digest() != m.get("sha256"):
        return "library bytes differ from the manifest"
    now = source_digests()
    was = m.get("sources", {})
    changed = sorted(k for k in set(now) | set(was) if now.get(k) != was.get(k))
    if changed:
        return "sources changed since the build: " + ", ".join(changed)
    return None


if __name__ == "__main__":
    build(verbose=True)
    print(LIB)
