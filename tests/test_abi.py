"""The C ABI of libarbor_hip.so on the CPU (no kernel is launched): the library loads and
exports every function include/arbor_sampling.h declares, the ctypes mirror of the params
struct matches the C layout, the header's constants match the host module's, and every
argument check returns its documented status before any device work."""
from __future__ import annotations

import ctypes
import re
import subprocess

import numpy as np
import pytest

from arbornet_amd import sampling as S
from arbornet_amd import synthetic as syn

HEADER = S.HEADER_PATH.read_text()


def _defines() -> dict[str, int]:
    out = {}
    for name, val in re.findall(r"#define\s+(ARBOR_[A-Z0-9_]+)\s+\(?(-?\d+)u?\)?", HEADER):
        out[name] = int(val)
    return out


def test_library_exports_every_header_function():
    names = S.header_functions()
    assert {"arbor_sample", "arbor_sample_workspace_bytes", "arbor_sampling_params_init", "arbor_abi_version",
            "arbor_last_error"} <= set(names)
    lib = S.library()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    nm = subprocess.run(["nm", "-D", "--defined-only", str(S.LIB_PATH)], capture_output=True, text=True, check=True)
    exported = set(re.findall(r" T (arbor_\w+)$", nm.stdout, flags=re.M))
    assert set(names) <= exported
    assert exported <= set(names), f"exported but not declared: {exported - set(names)}"


def test_abi_version_and_constants():
    d = _defines()
    assert S.library().arbor_abi_version() == d["ARBOR_ABI_VERSION"]
    assert d["ARBOR_DTYPE_F32"] == S.ARBOR_DTYPE_F32 and d["ARBOR_DTYPE_BF16"] == S.ARBOR_DTYPE_BF16
    assert d["ARBOR_FLAG_WRITE_PROBS"] == S.ARBOR_FLAG_WRITE_PROBS
    for code, name in S.STATUS_NAMES.items():
        assert d[name] == code, name
    assert (d["ARBOR_ID_EMPTY"], d["ARBOR_ID_INVALID"], d["ARBOR_ID_BAD_HISTORY"], d["ARBOR_ID_STALLED"]) == (
        S.ARBOR_ID_EMPTY, S.ARBOR_ID_INVALID, S.ARBOR_ID_BAD_HISTORY, S.ARBOR_ID_STALLED)


def test_params_layout_matches_c(tmp_path):
    fields = [f for f, _ in S.SamplingParams._fields_]
    src = tmp_path / "layout.c"
    body = "".join(f'  printf("{f} %zu\\n", offsetof(arbor_sampling_params, {f}));\n' for f in fields)
    src.write_text("#include <stddef.h>\n#include <stdio.h>\n#include \"arbor_sampling.h\"\nint main(void) {\n"
                   "  printf(\"sizeof %zu\\n\", sizeof(arbor_sampling_params));\n" + body + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", str(S.HEADER_PATH.parent), str(src), "-o", str(exe)], check=True)
    out = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                        check=True).stdout.splitlines())
    assert int(out["sizeof"]) == ctypes.sizeof(S.SamplingParams)
    for f in fields:
        assert int(out[f]) == getattr(S.SamplingParams, f).offset, f


def test_params_init_defaults():
    p = S.SamplingParams()
    S.library().arbor_sampling_params_init(ctypes.byref(p), 7, 1000)
    assert p.struct_size == ctypes.sizeof(S.SamplingParams)
    assert (p.batch, p.vocab, p.ld_logits, p.dtype) == (7, 1000, 1000, S.ARBOR_DTYPE_F32)
    assert (p.temperature, p.repetition_penalty, p.frequency_penalty, p.presence_penalty) == (1.0, 1.0, 0.0, 0.0)
    assert (p.top_k, p.top_p, p.min_p, p.hist_len, p.mask_words, p.flags) == (0, 1.0, 0.0, 0, 32, 0)
    q = S.SamplingParams.make(7, 1000)
    assert p.as_dict() == q.as_dict()


BAD = [
    (dict(struct_size=12), -2),
    (dict(batch=0), -3),
    (dict(vocab=0), -3),
    (dict(vocab=1 << 20, ld_logits=1 << 20), -3),
    (dict(ld_logits=999), -3),
    (dict(dtype=2), -4),
    (dict(temperature=0.0), -5),
    (dict(temperature=float("inf")), -5),
    (dict(temperature=float("nan")), -5),
    (dict(repetition_penalty=0.0), -6),
    (dict(frequency_penalty=float("nan")), -6),
    (dict(presence_penalty=float("-inf")), -6),
    (dict(top_k=-1), -7),
    (dict(top_p=0.0), -8),
    (dict(top_p=1.5), -8),
    (dict(min_p=1.0), -9),
    (dict(min_p=-0.1), -9),
    (dict(hist_len=-1), -10),
    (dict(hist_len=4097), -10),
    (dict(flags=2), -13),
]


@pytest.mark.parametrize("kw,status", BAD, ids=[f"{list(k)[0]}={list(k.values())[0]}" for k, _ in BAD])
def test_invalid_params_rejected(kw, status):
    p = S.SamplingParams.make(4, 1000)
    for k, v in kw.items():
        setattr(p, k, v)
    lib = S.library()
    assert lib.arbor_sample_workspace_bytes(ctypes.byref(p)) == 0
    st = S.sample_raw(p, 16, None, None, 16, 16, None, 16, 1 << 30, None)
    assert st == status
    assert lib.arbor_last_error()  # a message is always left


def test_null_params():
    lib = S.library()
    assert lib.arbor_sample(None, 16, None, None, 16, 16, None, 16, 1 << 30, None) == -1
    assert lib.arbor_sample_workspace_bytes(None) == 0


def test_argument_checks_before_launch():
    p = S.SamplingParams.make(4, 1000, hist_len=8)
    need = S.workspace_bytes(p)
    assert need > 0
    # required pointers
    assert S.sample_raw(p, None, 16, None, 16, 16, None, 16, need, None) == -1
    assert S.sample_raw(p, 16, 16, None, None, 16, None, 16, need, None) == -1
    assert S.sample_raw(p, 16, 16, None, 16, None, None, 16, need, None) == -1
    # history required when hist_len > 0
    assert S.sample_raw(p, 16, None, None, 16, 16, None, 16, need, None) == -10
    # mask words
    q = S.SamplingParams.make(4, 1000, mask_words=31)
    assert S.sample_raw(q, 16, None, 16, 16, 16, None, 16, S.workspace_bytes(q), None) == -11
    # probs flag without out_probs
    q = S.SamplingParams.make(4, 1000, flags=S.ARBOR_FLAG_WRITE_PROBS)
    assert S.sample_raw(q, 16, None, None, 16, 16, None, 16, S.workspace_bytes(q), None) == -13
    # workspace
    assert S.sample_raw(p, 16, 16, None, 16, 16, None, None, need, None) == -12
    assert S.sample_raw(p, 16, 16, None, 16, 16, None, 16, need - 1, None) == -12
    assert b"workspace" in S.library().arbor_last_error()


@pytest.mark.parametrize("name", sorted(syn.CONFIGS))
def test_workspace_bytes_configs(name):
    w = syn.CONFIGS[name]
    p = S.params_for(w)
    need = S.workspace_bytes(p)
    if name == "c2":
        # nucleus kernel, rows split over workgroups: one ~26 KB record per workgroup (at most
        # one workgroup per compute unit) and two barrier words per row
        assert 0 < need <= 256 * (26 << 10) + 16 * w.batch + 1024
    else:
        # streamed rows: at most the chunk lists of one workgroup per compute unit (520 B each)
        assert 0 < need <= 256 * 520 + 1024
    p.flags = S.ARBOR_FLAG_WRITE_PROBS
    assert S.workspace_bytes(p) > 0


def test_error_raises_with_status_name():
    with pytest.raises(S.ArborSamplingError, match="ARBOR_ERR_TEMPERATURE") as e:
        S.check(S.sample_raw(S.SamplingParams.make(1, 10, temperature=-1.0), 16, None, None, 16, 16, None, 16,
                             1 << 20, None))
    assert e.value.status == -5


def test_sampling_rejects_host_tensors():
    import torch

    with pytest.raises(S.ArborSamplingError) as e:
        S.Sampling.sample(torch.zeros(2, 10), torch.zeros(2))
    assert e.value.status == -14


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(S, "LIB_PATH", tmp_path / "absent.so")
    monkeypatch.setattr(S, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        S.library()


def test_product_does_not_use_the_oracle():
    """Nothing under arbornet_amd/ imports, loads or names the CPU oracle."""
    pkg = S.LIB_PATH.parent
    for f in list(pkg.rglob("*.py")) + list(pkg.rglob("*.hip")) + list(pkg.rglob("*.hpp")) + list(pkg.rglob("*.c")):
        text = f.read_text()
        assert not re.search(r"import\s+oracle|from\s+oracle|liboracle|oracle[/.]|sampling_oracle", text), \
            f"{f} refers to the oracle"


def test_device_count_without_gpu():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a HIP device is visible")
    n = ctypes.c_int(-1)
    st = S.library().arbor_device_count(ctypes.byref(n))
    assert n.value == 0 and st != 0


def test_params_for_matches_workload():
    w = syn.CONFIGS["c3"]
    p = S.params_for(w)
    assert (p.batch, p.vocab, p.top_k, p.hist_len) == (256, 128256, 50, 1024)
    assert np.float32(p.top_p) == np.float32(0.95)


def test_sample_append_argument_checks():
    # rejected before anything reaches the device
    lib = S.library()
    p = S.SamplingParams.make(4, 1000, hist_len=8)
    need = S.workspace_bytes(p)
    assert S.sample_append_raw(p, 16, None, 16, None, 16, 16, None, 16, need, None) == -10  # no ring
    assert S.sample_append_raw(p, 16, 16, None, None, 16, 16, None, 16, need, None) == -10  # no positions
    q = S.SamplingParams.make(4, 1000)  # hist_len 0: nothing to append to
    assert S.sample_append_raw(q, 16, 16, 16, None, 16, 16, None, 16, S.workspace_bytes(q), None) == -10
    r = S.SamplingParams.make(4, 1000, hist_len=8, top_p=2.0)
    assert S.sample_append_raw(r, 16, 16, 16, None, 16, 16, None, 16, 1 << 30, None) == -8
    assert lib.arbor_sample_append(None, 16, 16, 16, None, 16, 16, None, 16, 1 << 30, None) == -1
    assert b"history" in lib.arbor_last_error() or lib.arbor_last_error()


def test_lm_head_arguments_checked_on_the_host():
    # the LM head's shape, dtype and layout rules, checked before anything is launched
    lib = S.library()
    assert lib.arbor_lm_head_packed_bytes(4096, 128256) == ((128256 + 255) // 256 * 256) * 4096 * 2
    assert lib.arbor_lm_head_packed_bytes(100, 1000) == 0        # hidden not a multiple of 128
    assert lib.arbor_lm_head_packed_bytes(128, 0) == 0
    assert lib.arbor_lm_head_packed_bytes(128, S.ARBOR_VOCAB_MAX + 1) == 0
    assert lib.arbor_lm_head_pack(16, 0, 0, 100, 1000, 16, None) == -3      # ARBOR_ERR_SHAPE
    assert lib.arbor_lm_head_pack(16, 7, 0, 128, 1000, 16, None) == -4      # ARBOR_ERR_DTYPE
    assert lib.arbor_lm_head_pack(16, 0, 2, 128, 1000, 16, None) == -13     # unknown layout
    assert lib.arbor_lm_head_pack(None, 0, 0, 128, 1000, 16, None) == -1    # ARBOR_ERR_NULL
    assert lib.arbor_lm_head(16, 1, 4, 120, 16, None, 128, 1000, 1.0, 16, 0, 1000, None, None) == -3  # ld_x < hidden
    assert lib.arbor_lm_head(16, 1, 4, 128, 16, None, 128, 1000, 1.0, 16, 3, 1000, None, None) == -4  # logits dtype
    assert lib.arbor_lm_head(16, 1, 4, 128, 16, None, 128, 1000, float("inf"), 16, 0, 1000, None, None) == -5
    assert lib.arbor_lm_head(None, 1, 4, 128, 16, None, 128, 1000, 1.0, 16, 0, 1000, None, None) == -1
    assert lib.arbor_lm_head(8, 1, 4, 128, 16, None, 128, 1000, 1.0, 16, 0, 1000, None, None) == -3  # x not 16-byte aligned
    assert lib.arbor_lm_head(None, 1, 0, 128, None, None, 128, 1000, 1.0, None, 0, 1000, None, None) == 0  # empty batch
