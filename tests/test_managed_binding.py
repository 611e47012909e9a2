"""The managed (C#) side of the boundary against the C header, on the CPU: every function
include/arbor_sampling.h declares has a DllImport in ArborHip.cs with the same name, the same
parameter order and marshalling types that match the C types, the C# params struct has the
header's fields in the header's order with matching types, and the C# constants equal the
header's. (No .NET toolchain exists here to compile the C# files; this is the check the
P/Invoke declarations of the reference, ArborNet.Core/Native/PInvoke/CUDA.cs:90-202, never
had.)"""
from __future__ import annotations

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = (ROOT / "include" / "arbor_sampling.h").read_text()
DOTNET = ROOT / "arbornet_amd" / "dotnet" / "ArborNet.Core"
CS = (DOTNET / "Native" / "PInvoke" / "ArborHip.cs").read_text()


def _strip_c_comments(s: str) -> str:
    return re.sub(r"/\*.*?\*/", "", s, flags=re.S)


def c_functions() -> dict[str, tuple[str, list[str]]]:
    """name -> (return type, [parameter types]) of the header's prototypes."""
    text = _strip_c_comments(HEADER)
    out = {}
    for m in re.finditer(r"^\s*((?:const\s+)?[a-z_0-9]+\s*\**)\s*(arbor_[a-z_0-9]+)\s*\(([^)]*)\)\s*;", text, re.M):
        ret, name, args = m.group(1), m.group(2), m.group(3)
        params = []
        for a in [x.strip() for x in args.split(",")]:
            if a in ("", "void"):
                continue
            a = re.sub(r"\s*\b[a-z_0-9]+$", "", a)  # drop the parameter name
            params.append(re.sub(r"\s+", " ", a.replace("*", " *")).strip())
        out[name] = (re.sub(r"\s+", " ", ret.replace("*", " *")).strip(), params)
    return out


def cs_functions() -> dict[str, tuple[str, list[str]]]:
    out = {}
    for m in re.finditer(r"\[DllImport\([^\]]*\)\]\s*public static extern\s+(\w+)\s+(arbor_\w+)\s*\(([^)]*)\)\s*;",
                         CS, re.S):
        ret, name, args = m.group(1), m.group(2), m.group(3)
        params = []
        for a in [x.strip() for x in args.split(",") if x.strip()]:
            toks = a.split()
            params.append(" ".join(toks[:-1]))  # modifiers + type, without the name
        out[name] = (ret, params)
    return out


def c_to_cs(c: str, *, ret: bool = False) -> set[str]:
    """The marshalling types a C# declaration may use for a C type."""
    c = c.replace("const ", "")
    table = {
        "int": {"int"}, "int32_t": {"int"}, "uint32_t": {"uint"}, "size_t": {"UIntPtr", "nuint"}, "float": {"float"},
        "void": {"void"}, "char *": {"IntPtr"},
        "arbor_sampling_params *": {"ref ArborSamplingParams", "out ArborSamplingParams"},
        "int *": {"out int", "IntPtr"}, "void * *": {"out IntPtr"},
    }
    if c in table:
        return table[c]
    if c.endswith("*"):
        return {"IntPtr"}  # device pointers and other buffers
    raise KeyError(c)


def test_every_header_function_has_a_matching_dllimport():
    cf, sf = c_functions(), cs_functions()
    assert set(cf) == set(sf), f"header only: {set(cf) - set(sf)}, C# only: {set(sf) - set(cf)}"
    for name, (cret, cparams) in cf.items():
        sret, sparams = sf[name]
        assert sret in c_to_cs(cret, ret=True), (name, cret, sret)
        assert len(cparams) == len(sparams), (name, cparams, sparams)
        for i, (c, s) in enumerate(zip(cparams, sparams)):
            assert s in c_to_cs(c), f"{name} parameter {i}: C {c!r} bound as {s!r}"


def test_params_struct_fields_in_order():
    body = re.search(r"typedef struct arbor_sampling_params \{(.*?)\} arbor_sampling_params;",
                     _strip_c_comments(HEADER), re.S).group(1)
    cfields = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        ctype, names = decl.split(None, 1)
        cfields += [(ctype, n.strip()) for n in names.split(",")]
    sbody = re.search(r"public struct ArborSamplingParams\s*\{(.*?)\}", CS, re.S).group(1)
    sfields = re.findall(r"public\s+(\w+)\s+(\w+);", sbody)
    assert len(cfields) == len(sfields)
    ctype_cs = {"uint32_t": "uint", "int32_t": "int", "float": "float"}
    for (ct, cn), (st, sn) in zip(cfields, sfields):
        assert sn == "".join(w.capitalize() for w in cn.split("_")), (cn, sn)
        assert st == ctype_cs[ct], (cn, ct, st)
    assert re.search(r"\[StructLayout\(LayoutKind\.Sequential\)\]\s*public struct ArborSamplingParams", CS)


def test_constants_match_the_header():
    defines = {n: int(v) for n, v in re.findall(r"#define\s+(ARBOR_[A-Z0-9_]+)\s+\(?(-?\d+)u?\)?\s*(?:/\*|$)",
                                                HEADER, re.M)}
    consts = {n: v for n, v in re.findall(r"public const (?:int|uint) (ARBOR_[A-Z0-9_]+) = ([^;]+);", CS)}
    for name, val in defines.items():
        assert name in consts, f"{name} missing in ArborHip.cs"
        assert eval(consts[name].replace("u", "")) == val, (name, consts[name], val)  # noqa: S307 (literal ints)
    scratch = re.search(r"#define ARBOR_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", HEADER)
    assert eval(consts["ARBOR_NOALLOC_SCRATCH_BYTES"].replace("u", "")) == int(scratch.group(1)) << int(scratch.group(2))


@pytest.mark.parametrize("path", sorted(p.relative_to(DOTNET).as_posix() for p in DOTNET.rglob("*.cs")))
def test_managed_sources_are_balanced(path):
    # no compiler here: at least every brace, bracket and parenthesis closes, and each file
    # declares one namespace of ArborNet.Core
    src = (DOTNET / path).read_text()
    code = re.sub(r'"(?:\\.|[^"\\])*"', '""', re.sub(r"//[^\n]*", "", src))
    for o, c in ("{}", "()", "[]"):
        assert code.count(o) == code.count(c), (path, o)
    assert re.search(r"^namespace ArborNet\.Core(\.\w+)*$", src, re.M), path


def test_calls_use_declared_entry_points():
    # every ArborHip.<entry point> the managed op calls is declared
    sf = cs_functions()
    for p in DOTNET.rglob("*.cs"):
        for name in re.findall(r"ArborHip\.(arbor_\w+)\(", p.read_text()):
            assert name in sf, (p.name, name)
