"""The gfx950 route in routing data: registry rows and planner admission.

The reference certifies a GPU route per artifact in its support registry
(``src/toktier/routing/tables/support_registry.v1.json``: ``artifacts[*].
backends.gpu.deliveries.prebuilt`` with ``status``, ``devices``,
``binary_digest``, ``toolchain``, ``driver_min``) and admits it at plan
time with the checks of ``src/toktier/routing/plan.py:1-39`` (steps 3-5
and 9-13 for a prebuilt GPU delivery, ``:211-324``, ``:470-580``;
``registry_view.py:192-206`` for the per-architecture status labels).
This module gives the gfx950 engine the same two halves:

- rows: one per artifact the engine has been judged on, bound to the code
  object by the library's build key (sources, hipcc flags, hipcc version;
  ``toktier_amd/_lib/manifest.json``) and to the device by
  ``devices: ["gfx950"]``; the status is ``certified`` only when the GPU
  parity suite passed on that very build on a gfx950 device (the evidence
  file the suite writes), else ``experimental``;
- admission: the same ordered checks and reason codes, each refusal marked
  waivable or not as the reference marks it; the ``experimental`` policy
  proceeds past waivable refusals and records them as waivers, the
  ``certified`` policy does not.

There is no CPU engine behind this path, so a route that is not admitted is
an error for the caller (``certified`` policy) rather than a fallback.
"""

from __future__ import annotations

import hashlib
import json
import sys
from dataclasses import dataclass, field
from pathlib import Path

REGISTRY_PATH = (Path(__file__).resolve().parent / "data" / "registry" /
                 "gfx950_routes.v1.json")
EVIDENCE_PATH = REGISTRY_PATH.with_name("gfx950_evidence.v1.json")
SCHEMA_VERSION = 1
ARCH = "gfx950"
ORACLE = {"id": "tokenizers", "version": "0.22.2"}

STATUS_CERTIFIED = "certified"
STATUS_EXPERIMENTAL = "experimental"
STATUS_UNSUPPORTED = "unsupported"
ELIGIBLE_STATUSES = (STATUS_CERTIFIED,)

POLICY_CERTIFIED = "certified"
POLICY_EXPERIMENTAL = "experimental"

# reason codes of the reference planner (plan.py:13-27)
R_BACKEND_UNAVAILABLE = "R_BACKEND_UNAVAILABLE"
R_NO_GPU_DETECTED = "R_NO_GPU_DETECTED"
R_UNCERTIFIED_ARTIFACT = "R_UNCERTIFIED_ARTIFACT"
R_ORACLE_MISMATCH = "R_ORACLE_MISMATCH"
R_SM_UNCERTIFIED = "R_SM_UNCERTIFIED"
R_DRIVER_TOO_OLD = "R_DRIVER_TOO_OLD"
R_KERNEL_BUILD_FAILED = "R_KERNEL_BUILD_FAILED"
R_KERNEL_DIGEST_MISMATCH = "R_KERNEL_DIGEST_MISMATCH"


@dataclass(frozen=True)
class Facts:
    """What the engine observed about this process and device."""

    library_loaded: bool
    build_key: str | None          # manifest build key of the loaded library
    build_failed: bool
    architectures: tuple[str, ...]  # of the devices the probe saw
    driver_version: int | None      # hipDriverGetVersion
    oracle_version: str | None = ORACLE["version"]
    # why the loaded library is not the build the manifest names (its bytes
    # differ, or the sources changed since it was built); None when it is
    build_mismatch: str | None = None


@dataclass(frozen=True)
class Reason:
    code: str
    waivable: bool
    detail: dict = field(default_factory=dict)

    def as_dict(self) -> dict:
        return {"code": self.code, "waivable": self.waivable, **self.detail}


@dataclass(frozen=True)
class Admission:
    """``admitted``: the gfx950 route runs; ``refusals``: reasons it would
    not run under the certified policy; ``waivers``: those the experimental
    policy proceeded past."""

    admitted: bool
    policy: str
    refusals: tuple[Reason, ...]
    waivers: tuple[Reason, ...]
    row: dict | None

    def as_dict(self) -> dict:
        row = self.row or {}
        return {
            "admitted": self.admitted, "policy": self.policy,
            "refusals": [r.as_dict() for r in self.refusals],
            "waivers": [r.as_dict() for r in self.waivers],
            "status": row.get("status"),
            "devices": row.get("devices"),
            "binary_digest": row.get("binary_digest"),
            "evidence_id": row.get("evidence_id"),
        }


def load_registry(path: Path = REGISTRY_PATH) -> dict:
    reg = json.loads(Path(path).read_text())
    if reg.get("schema_version") != SCHEMA_VERSION:
        raise ValueError(f"{path}: schema_version {reg.get('schema_version')}")
    for a in reg.get("artifacts", []):
        for key in ("artifact_sha256", "family", "backends"):
            if key not in a:
                raise ValueError(f"{path}: artifact row without {key}")
    if reg.get("root_digest") != root_digest(reg):
        raise ValueError(f"{path}: root digest does not match its rows")
    return reg


def root_digest(reg: dict) -> str:
    body = json.dumps(reg.get("artifacts", []), sort_keys=True,
                      separators=(",", ":"))
    return "sha256:" + hashlib.sha256(b"toktier-gfx950-registry\0" +
                                      body.encode()).hexdigest()


def prebuilt_row(reg: dict, artifact_sha256: str) -> tuple[dict | None, dict | None]:
    """(artifact record, its gpu prebuilt row) or Nones."""
    for a in reg.get("artifacts", []):
        if a["artifact_sha256"] == artifact_sha256:
            gpu = a["backends"].get("gpu") or {}
            return a, (gpu.get("deliveries") or {}).get("prebuilt")
    return None, None


def architecture_statuses(row: dict) -> dict[str, str]:
    """Per-architecture labels: judged devices carry the row's status,
    shipped-but-unjudged ones are ``experimental`` (registry_view.py:
    192-206)."""
    out = {d: row["status"] for d in row.get("devices", [])}
    for d in row.get("devices_experimental", []):
        out.setdefault(d, STATUS_EXPERIMENTAL)
    return out


def admit(reg: dict | None, artifact_sha256: str, facts: Facts,
          policy: str = POLICY_EXPERIMENTAL) -> Admission:
    """The reference planner's checks for a prebuilt GPU delivery, in its
    order (plan.py:1-39). The first refusal that is not waivable, or under
    the certified policy the first refusal of any kind, ends the route."""
    if policy not in (POLICY_CERTIFIED, POLICY_EXPERIMENTAL):
        raise ValueError(f"unknown policy {policy!r}")
    refusals: list[Reason] = []

    def refuse(code: str, waivable: bool, **detail) -> bool:
        refusals.append(Reason(code, waivable, detail))
        return waivable and policy == POLICY_EXPERIMENTAL

    def verdict(row, admitted):
        waivers = tuple(r for r in refusals) if admitted else ()
        return Admission(admitted, policy, tuple(refusals), waivers, row)

    # 3. the backend has to exist
    if not facts.library_loaded:
        refuse(R_BACKEND_UNAVAILABLE, False, module="libtoktier_hip.so")
        return verdict(None, False)
    # 4. and something to run on
    if not facts.architectures:
        refuse(R_NO_GPU_DETECTED, False)
        return verdict(None, False)
    # 5. certification identity and status
    rec, row = prebuilt_row(reg or {}, artifact_sha256)
    if rec is None or row is None:
        ok = refuse(R_UNCERTIFIED_ARTIFACT, True,
                    cause="no_record" if rec is None else "no_backend_entry",
                    artifact_sha256=artifact_sha256)
        return verdict(None, ok)
    if row["status"] == STATUS_UNSUPPORTED:
        refuse(R_UNCERTIFIED_ARTIFACT, False, cause="status_unsupported")
        return verdict(row, False)
    if row["status"] not in ELIGIBLE_STATUSES:
        if not refuse(R_UNCERTIFIED_ARTIFACT,
                      row["status"] == STATUS_EXPERIMENTAL,
                      cause="status_not_eligible", status=row["status"]):
            return verdict(row, False)
    # 7. oracle version inside the certified set
    want = rec.get("oracle_version")
    if want and facts.oracle_version != want:
        if not refuse(R_ORACLE_MISMATCH, True, expected=want,
                      observed=facts.oracle_version):
            return verdict(row, False)
    # 9. device architecture explicitly judged
    devices = row.get("devices", [])
    if devices and not set(facts.architectures) & set(devices):
        if not refuse(R_SM_UNCERTIFIED, True,
                      observed=sorted(facts.architectures), certified=devices):
            return verdict(row, False)
    # 10. driver at or above the certified floor
    floor = row.get("driver_min")
    if floor is not None and (facts.driver_version is None or
                              facts.driver_version < int(floor)):
        if not refuse(R_DRIVER_TOO_OLD, True, installed=facts.driver_version,
                      required=floor):
            return verdict(row, False)
    # 11. a build that failed leaves nothing to run (never waived)
    if facts.build_failed:
        refuse(R_KERNEL_BUILD_FAILED, False)
        return verdict(row, False)
    # 12. bound digest: the code object the row was judged on (a library
    # that is not the manifest's build, or sources edited after it, carry
    # no judged digest at all)
    if facts.build_mismatch is not None:
        if not refuse(R_KERNEL_DIGEST_MISMATCH, True,
                      expected_digest=row.get("binary_digest"),
                      observed_digest=None, cause=facts.build_mismatch):
            return verdict(row, False)
    elif row.get("binary_digest") != facts.build_key:
        if not refuse(R_KERNEL_DIGEST_MISMATCH, True,
                      expected_digest=row.get("binary_digest"),
                      observed_digest=facts.build_key):
            return verdict(row, False)
    return verdict(row, True)


# ------------------------------------------------------- generating rows

def suite_judged(evidence: dict, manifest: dict) -> bool:
    """The evidence is a complete, clean run of the GPU suite on this very
    build on gfx950: the library was the manifest's build, the whole
    ``-m gpu`` selection ran (no ``-k``, nothing deselected), and no test
    failed or was skipped (tests parked in the source by an explicit skip
    mark with a reason are listed by node id under ``parked`` and counted
    as collected, not as run; each blocks the family it covers,
    ``family_judged``)."""
    sel = evidence.get("selection") or {}
    ran = (evidence.get("passed", 0) + evidence.get("failed", 0)
           + evidence.get("skipped", 0) + len(evidence.get("parked") or []))
    return (evidence.get("build_key") == manifest["build_key"]
            and evidence.get("build_mismatch") is None
            and evidence.get("architecture") == ARCH
            and evidence.get("failed", 1) == 0
            and evidence.get("skipped", 1) == 0
            and evidence.get("passed", 0) > 0
            and sel.get("complete") is True
            and sel.get("deselected_gpu", 1) == 0
            and sel.get("collected_gpu") == ran)


def family_judged(evidence: dict, manifest: dict, family: str) -> bool:
    """Certified for `family`: the suite as a whole is judged, the
    family's own parity tests ran and all passed, and none of them, nor
    any test shared by every family, is parked (a parked test is a case
    of the family that no run covered)."""
    fams = evidence.get("families") or {}
    fam = fams.get(family) or {}
    shared = fams.get("shared") or {}
    return (suite_judged(evidence, manifest)
            and fam.get("passed", 0) > 0
            and fam.get("failed", 1) == 0
            and fam.get("skipped", 1) == 0
            and fam.get("parked", 0) == 0
            and shared.get("parked", 0) == 0)


def generate(evidence: dict, manifest: dict, artifacts: dict[str, str]) -> dict:
    """Registry rows for `artifacts` (family -> artifact sha256) from the
    library manifest and the evidence the GPU parity suite wrote. A row is
    certified only when the whole suite ran clean on this build on gfx950
    (``suite_judged``) and the family's own tests ran and passed
    (``family_judged``); otherwise it is experimental."""
    rows = []
    for family, sha in sorted(artifacts.items()):
        judged = family_judged(evidence, manifest, family)
        status = STATUS_CERTIFIED if judged else STATUS_EXPERIMENTAL
        fam = (evidence.get("families") or {}).get(family) or {}
        rows.append({
            "artifact_sha256": sha,
            "family": family,
            "oracle_id": ORACLE["id"],
            "oracle_version": ORACLE["version"],
            "evidence_id": evidence.get("evidence_id"),
            "backends": {"gpu": {
                "status": status,
                "deliveries": {"prebuilt": {
                    "status": status,
                    "binary_digest": manifest["build_key"],
                    "toolchain": " / ".join(manifest.get("hipcc", [])),
                    "build_flags": manifest.get("flags", []),
                    "devices": [ARCH] if judged else [],
                    "devices_experimental": [] if judged else [ARCH],
                    "driver_min": evidence.get("driver_version"),
                    "readings": {k: fam.get(k) for k in
                                 ("passed", "failed", "skipped")},
                }},
            }},
        })
    reg = {"schema_version": SCHEMA_VERSION,
           "generated_by": {"tool": "toktier_amd.registry"},
           "artifacts": rows}
    reg["root_digest"] = root_digest(reg)
    return reg


def main(argv: list[str]) -> int:
    """``python -m toktier_amd.registry [evidence.json]``: rewrite the
    committed rows from an evidence file (default: the committed one)."""
    from . import standin
    from ._build import MANIFEST
    src = Path(argv[0]) if argv else EVIDENCE_PATH
    evidence = json.loads(src.read_text())
    if src != EVIDENCE_PATH:
        EVIDENCE_PATH.parent.mkdir(parents=True, exist_ok=True)
        EVIDENCE_PATH.write_text(json.dumps(evidence, indent=1, sort_keys=True) + "\n")
    manifest = json.loads(MANIFEST.read_text())
    reg = generate(evidence, manifest, dict(standin.ARTIFACT_SHA256))
    REGISTRY_PATH.write_text(json.dumps(reg, indent=1, sort_keys=True) + "\n")
    status = reg["artifacts"][0]["backends"]["gpu"]["status"] if reg["artifacts"] else None
    print(f"{REGISTRY_PATH}: {len(reg['artifacts'])} rows, status {status}")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
