"""The gfx950 route as the facade reports it: the engine's device facts
(architecture, driver, build key) against the committed registry rows."""

from __future__ import annotations

import json

import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["qwen3_8b", "llama_3_1_8b", "gpt2",
                                  "laguna_s_2_1", "deepseek_v3",
                                  "gpt_oss_120b", "kimi_k3"])
def test_route_admission(name):
    import toktier_amd
    from toktier_amd import registry
    from toktier_amd._build import MANIFEST
    t = toktier_amd.load(name)
    info = t.explain()
    adm = info["admission"]
    assert info["architectures"] == ["gfx950"] and adm["admitted"]
    assert t.engine.driver_version > 0
    build_key = json.loads(MANIFEST.read_text())["build_key"]
    row = None
    if registry.REGISTRY_PATH.exists():
        _, row = registry.prebuilt_row(registry.load_registry(),
                                       t.artifact_sha256)
    t.close()
    judged = (row is not None and row["status"] == registry.STATUS_CERTIFIED
              and row["binary_digest"] == build_key)
    if judged:
        # this build was certified on gfx950: the strict policy admits it
        strict = toktier_amd.load(name, policy="certified")
        assert strict.explain()["admission"]["refusals"] == []
        assert list(strict.encode("<|endoftext|> ok").array)
        strict.close()
    else:
        codes = {r["code"] for r in adm["waivers"]}
        assert codes & {registry.R_UNCERTIFIED_ARTIFACT,
                        registry.R_KERNEL_DIGEST_MISMATCH}
        with pytest.raises(toktier_amd.EngineError):
            toktier_amd.load(name, policy="certified")
