"""The committed gfx950 manifest entries (roost_amd/manifest.gfx950.toml) against the built library, by the rules
Roost's loader applies before it admits a kernel library: the SM entry (`KernelLibrary.Admit`,
`src/Starlings.Roost.Kernels/KernelLibrary.cs:375-399`), the one digest per SM library and the file's size and SHA-256
(`KernelLibrary.cs:402-420`, `VerifiedLibraryFile.cs:140-162`) and the three cross-check rules (`KernelLibrary.cs:343-373`).
Each rule is also shown to fail on a manifest that breaks it. CPU only: the registration table needs no device."""
import copy

import pytest
import tomli

import roost_amd
from roost_amd import manifest


@pytest.fixture(scope="module")
def lib():
    return roost_amd.KernelLibrary()


@pytest.fixture(scope="module")
def committed():
    return tomli.loads(manifest.MANIFEST_PATH.read_text())


def test_manifest_admits_the_built_library(lib, committed):
    regs = manifest.registrations(lib)
    assert len(regs) == len(lib.entries) >= 13
    manifest.cross_check(committed, regs)
    manifest.verify_binary(committed, lib.path)
    assert [s for s in committed["sm"] if s["arch"] == 950][0]["status"] in ("experimental", "supported")


def test_manifest_is_what_the_build_writes(lib, committed):
    """The committed file is the generator's output for this library: nothing was edited by hand."""
    assert manifest.render(lib, lib.path) == manifest.MANIFEST_PATH.read_text()


def test_manifest_schema_values(committed):
    """Op names from the C1 catalogue, flags and dtypes from the schema's enumerations, one binaries entry each."""
    for op in committed["ops"]:
        assert op["op"] in manifest.OP_NAMES.values()
        for v in op["variants"]:
            assert set(v["flags"]) <= {n for _, n in manifest.FLAG_NAMES}
            c = v["constraints"]
            assert c["sm_min"] == 950
            for key in ("act_dtypes", "kv_dtypes"):
                assert set(c.get(key, [])) <= set(manifest.DTYPE_NAMES)
            assert len(v["binaries"]) == 1 and v["binaries"][0]["arch"] == 950
    gdn = {v["id"]: v for op in committed["ops"] if op["op"] == "GatedDeltaRule" for v in op["variants"]}
    # The worker selects the recurrent variant by this id (reference CudaOps.cs:28).
    assert "gated-delta-rule-recurrent-aot" in gdn
    assert "needs_plan" not in gdn["gated-delta-rule-recurrent-aot"]["flags"]


def _variant(m, vid):
    return next(v for op in m["ops"] for v in op["variants"] if v["id"] == vid)


@pytest.mark.parametrize("change", ["unlisted variant", "flags differ", "sm_min differs", "listed but not registered",
                                    "no sm entry", "digest", "size", "two digests", "no binaries"])
def test_loader_rules_refuse_a_broken_manifest(lib, committed, change):
    m = copy.deepcopy(committed)
    regs = manifest.registrations(lib)
    if change == "unlisted variant":
        for op in m["ops"]:
            op["variants"] = [v for v in op["variants"] if v["id"] != "cache-write-gfx950"]
    elif change == "flags differ":
        _variant(m, "paged-attention-gfx950")["flags"].append("graph_capturable")
    elif change == "sm_min differs":
        _variant(m, "rope-gfx950")["constraints"]["sm_min"] = 90
    elif change == "listed but not registered":
        extra = copy.deepcopy(_variant(m, "rope-gfx950"))
        extra["id"] = "rope-gfx950-extra"
        next(op for op in m["ops"] if op["op"] == "Rope")["variants"].append(extra)
    elif change == "no sm entry":
        m["sm"] = [s for s in m["sm"] if s["arch"] != 950]
    elif change == "digest":
        for op in m["ops"]:
            for v in op["variants"]:
                v["binaries"][0]["sha256"] = "0" * 64
    elif change == "size":
        for op in m["ops"]:
            for v in op["variants"]:
                v["binaries"][0]["bytes"] += 1
    elif change == "two digests":
        _variant(m, "rope-gfx950")["binaries"][0]["sha256"] = "f" * 64
    elif change == "no binaries":
        for op in m["ops"]:
            for v in op["variants"]:
                v["binaries"] = []
    with pytest.raises(ValueError):
        manifest.cross_check(m, regs)
        manifest.verify_binary(m, lib.path)
