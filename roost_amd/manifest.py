"""The gfx950 entries of Roost's kernel manifest (contract C5), generated from the built library.

Roost's loader admits a kernel library only when the manifest (reference `kernels/manifest.toml`) has
- an `[[sm]]` entry for the library's arch (`KernelLibrary.Admit`, `src/Starlings.Roost.Kernels/KernelLibrary.cs:375-399`);
- a `[[ops.variants.binaries]]` entry for that arch naming one file size and SHA-256, which the loader checks before it
  maps the file (`KernelLibrary.ExpectedBinary`, `KernelLibrary.cs:402-420`; `VerifiedLibraryFile.cs:140-162`);
- every variant the library registers, with the same flags and `sm_min`, and no listed variant the library does not
  register (`KernelLibrary.CrossCheck`, `KernelLibrary.cs:343-373`).

`render()` writes those entries for this library: the `[[sm]]` entry for arch 950 and one `[[ops]]` block per op with
its variants (flags, constraints, binaries) read from the library's own registration table, so the manifest cannot
drift from what `roost_register` returns. The blocks append to the reference manifest unchanged: the loader keys
variants by (op, id) and reads only the binaries listed for the SM it loads. `cross_check()` and `verify_binary()`
restate the loader's three rules and its file check for the tests.
"""
from __future__ import annotations

import hashlib
from pathlib import Path

from . import abi

ARCH = 950
MANIFEST_NAME = "manifest.gfx950.toml"
MANIFEST_PATH = Path(__file__).resolve().parent / MANIFEST_NAME

# C1 op catalogue names (reference `src/Starlings.Roost.Abstractions/Abi/KernelAbi.cs:127-190`, `OpId`), which the
# manifest's `op` keys must use.
OP_NAMES = {
    1: "RmsNorm", 2: "QkNorm", 3: "Rope", 4: "PagedAttention", 5: "SiluAndMul", 6: "GeluAndMul", 7: "Gemm",
    8: "Embedding", 9: "LmHead", 10: "Residual", 11: "CacheWrite", 12: "CacheCopy", 13: "Argmax", 14: "Sample",
    64: "AddRmsNorm", 65: "AddRmsNormQuant", 66: "SiluMulQuant", 67: "QkvQkNormRopeCacheWrite",
    68: "GemmLoraEpilogue", 128: "GatedDeltaRule", 129: "CausalConv1d", 130: "RecurrentStateCopy",
    131: "RecurrentStateSnapshot", 132: "SlidingWindowAttention", 133: "GatedDeltaRuleGates", 134: "GatedRmsNorm",
    135: "SigmoidMul",
}
# Flag names of the manifest schema (`tools/kernel-manifest.schema.json`, `$defs/flag`) by ROOST_FLAG_* bit.
FLAG_NAMES = [(0x1, "graph_capturable"), (0x2, "deterministic"), (0x4, "batch_invariant"), (0x8, "needs_plan"),
              (0x10, "plan_per_shape")]
# ROOST_DTYPE_* ids 1..16 in order, by their schema names.
DTYPE_NAMES = ["f32", "f16", "bf16", "f64", "f8e4m3", "f8e5m2", "i8", "u8", "i16", "i32", "u32", "i64", "u64", "i4",
               "u4", "f4e2m1"]
LAYOUT_NAMES = ["row_major", "col_major", "paged_nhd", "paged_hnd"]


def flag_names(flags: int) -> list[str]:
    return [name for bit, name in FLAG_NAMES if flags & bit]


def flags_from_names(names) -> int:
    by_name = {name: bit for bit, name in FLAG_NAMES}
    out = 0
    for n in names:
        if n not in by_name:
            raise ValueError(f"unknown variant flag {n}")  # the reference parser refuses it too
        out |= by_name[n]
    return out


def _bits(mask: int, width: int) -> list[int]:
    return [i for i in range(width) if mask >> i & 1]


def constraints_table(c: abi.Constraints) -> dict:
    """RoostConstraints as the manifest's `[ops.variants.constraints]` keys. An all-ones mask (any head dim) is left
    out, as the reference manifest leaves out what a variant does not restrict."""
    t: dict = {"sm_min": int(c.sm_min)}
    if c.sm_max:
        t["sm_max"] = int(c.sm_max)
    if c.act_dtype_mask:
        t["act_dtypes"] = [DTYPE_NAMES[i - 1] for i in _bits(c.act_dtype_mask, 17) if i >= 1]
    if c.kv_dtype_mask:
        t["kv_dtypes"] = [DTYPE_NAMES[i - 1] for i in _bits(c.kv_dtype_mask, 17) if i >= 1]
    if c.head_dim_mask and c.head_dim_mask != (1 << 64) - 1:
        t["head_dims"] = [16 * (i + 1) for i in _bits(c.head_dim_mask, 64)]
    if c.page_size_mask:
        t["page_sizes"] = [1 << i for i in _bits(c.page_size_mask, 32)]
    if c.layout_mask:
        t["layouts"] = [LAYOUT_NAMES[i] for i in _bits(c.layout_mask, len(LAYOUT_NAMES))]
    t["min_alignment"] = int(c.min_alignment)
    if c.group_size_mask:
        t["group_sizes"] = [i + 1 for i in _bits(c.group_size_mask, 32)]
    return t


def registrations(lib) -> list[dict]:
    """(op, id, flags, constraints) of every entry `roost_register` returns, in table order."""
    return [{"op": OP_NAMES[e.op], "id": e.variant_id, "flags": int(e.flags), "sm_min": int(e.constraints.sm_min),
             "constraints": constraints_table(e.constraints)} for e in lib.entries]


def binary_of(path: Path) -> dict:
    data = Path(path).read_bytes()
    return {"arch": ARCH, "sha256": hashlib.sha256(data).hexdigest(), "bytes": len(data)}


def _value(v) -> str:
    if isinstance(v, str):
        return '"' + v + '"'
    if isinstance(v, list):
        return "[" + ", ".join(_value(x) for x in v) + "]"
    return str(v)


def render(lib, lib_path: Path) -> str:
    """The manifest entries of this build (TOML text)."""
    binary = binary_of(lib_path)
    lines = [
        "# gfx950 (MI355X) entries of the Roost kernel manifest (contract C5), written by roost_amd/build.py from the",
        "# library's own registration table and the built file; do not edit by hand. Append to kernels/manifest.toml:",
        "# the loader reads the [[sm]] entry for arch 950, checks the file against the binaries entry (size, SHA-256) and",
        "# cross-checks every registered (op, variant) against the variants listed here (flags and sm_min equal).",
        f"# Library: {Path(lib_path).name} (also linked as libroost_kernels_sm{ARCH}.so, the name the loader derives).",
        "",
        "[[sm]]",
        f"arch = {ARCH}",
        'status = "experimental"',
        'evidence = "tests/ (pytest -m gpu on an MI355X, parity against CpuOps) and profiles/"',
    ]
    by_op: dict[str, list[dict]] = {}
    for r in registrations(lib):
        by_op.setdefault(r["op"], []).append(r)
    for op, variants in by_op.items():
        lines += ["", "[[ops]]", f'op = "{op}"']
        for r in variants:
            lines += ["", "[[ops.variants]]", f'id = "{r["id"]}"', 'source = "roost"',
                      f"flags = {_value(flag_names(r['flags']))}", "", "[ops.variants.constraints]"]
            lines += [f"{k} = {_value(v)}" for k, v in r["constraints"].items()]
            lines += ["", "[[ops.variants.binaries]]", f"arch = {binary['arch']}", f'sha256 = "{binary["sha256"]}"',
                      f"bytes = {binary['bytes']}"]
    return "\n".join(lines) + "\n"


def write(lib, lib_path: Path, out: Path = MANIFEST_PATH) -> Path:
    text = render(lib, lib_path)
    if not out.exists() or out.read_text() != text:
        out.write_text(text)
    return out


# ---- The loader's rules, restated for the tests -------------------------------------------------------------------------

def listed_variants(manifest: dict, sm: int = ARCH) -> dict:
    """(op, id) -> (flags, sm_min, binaries) of the variants with a binaries entry for `sm`, as the loader builds its
    dictionary (`KernelLibrary.cs:345-347`; `KernelManifest.cs:173-207` for the fields)."""
    out = {}
    for op in manifest.get("ops", []):
        for v in op.get("variants", []):
            bins = [b for b in v.get("binaries", []) if b["arch"] == sm]
            if not bins:
                continue
            key = (op["op"], v["id"])
            if key in out:
                raise ValueError(f"{key} is listed twice for SM {sm}")
            out[key] = (flags_from_names(v.get("flags", [])), v.get("constraints", {}).get("sm_min", 0), bins)
    return out


def cross_check(manifest: dict, regs: list[dict], sm: int = ARCH) -> None:
    """`KernelLibrary.CrossCheck` (`KernelLibrary.cs:343-373`) and `Admit`'s SM lookup (`:386-391`): raises
    ValueError on the first mismatch."""
    if not any(s["arch"] == sm for s in manifest.get("sm", [])):
        raise ValueError(f"the manifest builds no library for SM {sm}")
    listed = listed_variants(manifest, sm)
    for r in regs:
        key = (r["op"], r["id"])
        if key not in listed:
            raise ValueError(f"the library registers {r['id']} ({r['op']}), which the manifest does not list for SM {sm}")
        flags, sm_min, _ = listed[key]
        if flags != r["flags"] or (sm_min != 0 and sm_min != r["sm_min"]):
            raise ValueError(f"{r['id']} ({r['op']}) registers flags {r['flags']} and sm_min {r['sm_min']}; "
                             f"the manifest says {flags} and {sm_min}")
    registered = {(r["op"], r["id"]) for r in regs}
    for key in listed:
        if key not in registered:
            raise ValueError(f"the manifest lists {key[1]} ({key[0]}) for SM {sm}, but the library does not register it")


def verify_binary(manifest: dict, path: Path, sm: int = ARCH) -> None:
    """`KernelLibrary.ExpectedBinary` (one digest for the SM's library) and `VerifiedLibraryFile`'s size and SHA-256
    check of the file (`KernelLibrary.cs:402-420`, `VerifiedLibraryFile.cs:140-162`)."""
    bins = [b for v in listed_variants(manifest, sm).values() for b in v[2]]
    if not bins:
        raise ValueError(f"no variant has a library digest for SM {sm}")
    digests = {b["sha256"].lower() for b in bins}
    if len(digests) != 1:
        raise ValueError(f"the manifest lists {len(digests)} different digests for the one SM {sm} library")
    expected = next((b for b in bins if b.get("bytes", 0)), bins[0])
    data = Path(path).read_bytes()
    if expected.get("bytes", 0) and len(data) != expected["bytes"]:
        raise ValueError(f"{path} has {len(data)} bytes; the manifest says {expected['bytes']}")
    if hashlib.sha256(data).hexdigest() != expected["sha256"].lower():
        raise ValueError(f"{path}: SHA-256 differs from the manifest's")
