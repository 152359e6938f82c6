"""Drop-in check of the C++ header API (CPU, compile-only): the reference's own callers of the
attention kernels -- src/engine/attention.hip, tests/test_attn_splitk.hip and
bench/attention/*.hip -- of the engine's attention layer through the drop-in
miso_amd/engine/attention.hpp -- src/engine/model.hip, tests/test_attention.hip (which reads the
scratch members) and bench/attention/bench_attention.hip -- and of the Q4_K / Q6_K GEMVs and prefill GEMMs -- src/engine/weights.hip,
tests/test_q4k_gemv.hip, tests/test_q6k_gemv.hip, tests/test_gemv_dispatch.hip,
tests/test_qgemm.hip -- compile UNCHANGED for gfx950 with this repository's miso_amd/kernels
ahead of the reference's kernels/ on the include path, and the preprocessor really picks this repository's headers (while the
reference's own rmsnorm.hpp and wave.hpp stay reachable in the same translation unit without
clashes).

Runs only where the reference tree and hipcc exist (this container); nothing is copied, objects
go to a temporary directory.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
REF = Path("/root/reference")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# (caller, the header of ours it includes itself, or None if only through engine headers)
CALLERS = [
    ("src/engine/attention.hip", "attention_decode.hpp"),
    ("tests/test_attn_splitk.hip", "attention_decode.hpp"),
    ("bench/attention/bench_combine.hip", "attention_decode.hpp"),
    ("bench/attention/bench_attention.hip", None),  # only through engine/attention.hpp
    ("tests/test_q4k_gemv.hip", "q4k_gemv.hpp"),
    ("tests/test_q6k_gemv.hip", "q6k_gemv.hpp"),
    ("tests/test_gemv_dispatch.hip", "mixed_gemv.hpp"),
    ("tests/test_qgemm.hip", "qgemm.hpp"),
    ("src/engine/weights.hip", "qgemm.hpp"),
]

# The engine drop-in (miso_amd/engine/attention.{hpp,hip}): the reference's src/engine/model.hip
# compiles unchanged with it in place of src/engine/attention.hpp, and the drop-in's own source
# compiles against the engine's headers.
ENGINE = ROOT / "miso_amd"
OURS = ("attention_decode.hpp", "attention_prefill.hpp", "q4k_gemv.hpp", "q6k_gemv.hpp",
        "mixed_gemv.hpp", "qgemm.hpp")

pytestmark = pytest.mark.skipif(not (REF / "kernels").is_dir() or not Path(HIPCC).exists(),
                                reason="reference tree or hipcc not available")


@pytest.mark.parametrize("caller,direct", CALLERS)
def test_reference_caller_compiles_against_our_headers(caller, direct, tmp_path):
    src = REF / caller
    cmd = [HIPCC, "-std=c++20", "-O1", "--offload-arch=gfx950", "-c", str(src),
           "-o", str(tmp_path / "x.o"), "-H",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I", str(ROOT / "miso_amd" / "kernels"),
           "-I", str(REF / "kernels"), "-I", str(REF / "src"),
           "-isystem", str(REF / "third_party"),
           '-DMISO_ORNITH_GGUF="/nonexistent.gguf"', '-DMISO_FIXTURE_DIR="/nonexistent"',
           '-DMISO_GOLDEN_DIR="/nonexistent"']
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-4000:]
    included = [l.lstrip(". ").strip() for l in res.stderr.splitlines() if l.startswith(".")]
    ours = str(ROOT / "miso_amd" / "kernels")
    for name in OURS:
        hits = [p for p in included if p.endswith("/" + name)]
        if hits:  # every resolution of these headers is ours
            assert all(Path(p).resolve().as_posix().startswith(ours) for p in hits), hits
    if direct:
        assert any(p.endswith("/" + direct) for p in included)


def _hipcc(src, tmp_path, includes, defines=()):
    cmd = [HIPCC, "-std=c++20", "-O1", "--offload-arch=gfx950", "-c", str(src),
           "-o", str(tmp_path / "x.o"), "-H",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           *[a for inc in includes for a in ("-I", str(inc))],
           "-isystem", str(REF / "third_party"), *defines]
    return subprocess.run(cmd, capture_output=True, text=True, timeout=600)


def test_engine_model_compiles_with_the_attention_drop_in(tmp_path):
    res = _hipcc(REF / "src/engine/model.hip", tmp_path,
                 [ENGINE, ROOT / "miso_amd" / "kernels", REF / "kernels", REF / "src"])
    assert res.returncode == 0, res.stderr[-4000:]
    included = [l.lstrip(". ").strip() for l in res.stderr.splitlines() if l.startswith(".")]
    hits = [p for p in included if p.endswith("engine/attention.hpp")]
    assert hits and all(Path(p).resolve().as_posix().startswith(str(ENGINE)) for p in hits), hits


# The reference's callers of the engine's attention API, which read the scratch members
# (tests/test_attention.hip:68 `scratch.core`, :104 `ps.core`) and construct the scratch types
# (bench/attention/bench_attention.hip:17): unchanged, with the drop-in picked over
# src/engine/attention.hpp.
ENGINE_CALLERS = ["tests/test_attention.hip", "bench/attention/bench_attention.hip"]


@pytest.mark.parametrize("caller", ENGINE_CALLERS)
def test_engine_callers_compile_with_the_attention_drop_in(caller, tmp_path):
    res = _hipcc(REF / caller, tmp_path,
                 [ENGINE, ROOT / "miso_amd" / "kernels", REF / "kernels", REF / "src"],
                 ['-DMISO_ORNITH_GGUF="/nonexistent.gguf"', '-DMISO_GOLDEN_DIR="/nonexistent"'])
    assert res.returncode == 0, res.stderr[-4000:]
    included = [l.lstrip(". ").strip() for l in res.stderr.splitlines() if l.startswith(".")]
    hits = [p for p in included if p.endswith("engine/attention.hpp")]
    assert hits and all(Path(p).resolve().as_posix().startswith(str(ENGINE)) for p in hits), hits


def test_attention_drop_in_compiles_against_the_engine_headers(tmp_path):
    res = _hipcc(ENGINE / "engine" / "attention.hip", tmp_path,
                 [ENGINE, ROOT / "miso_amd" / "kernels", REF / "kernels", REF / "src"])
    assert res.returncode == 0, res.stderr[-4000:]
