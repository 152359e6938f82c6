"""The engine-constant sweep (miso_amd.retune): argument handling on the CPU, a quick sweep on
the GPU through the same C ABI entry points the engine's attention calls use."""
import pytest


def test_retune_importable_and_documented():
    from miso_amd import retune
    assert "kMaxSplits" in retune.__doc__ and "kMaxChunk" in retune.__doc__
    assert retune.PROJ == 8192 + 512 + 512


@pytest.mark.gpu
def test_retune_quick_runs():
    from miso_amd import retune
    out = retune.run(quick=True)
    assert [r["ctx"] for r in out["max_splits"]] == [512, 4096]
    for r in out["max_splits"]:
        assert r["cap60"]["n_splits"] <= 60 and r["cap128"]["n_splits"] <= 128
        assert r["cap60"]["us"] > 0 and r["cap128"]["us"] > 0
    assert [r["chunk"] for r in out["chunk"]["rows"]] == [512, 2048]
    assert all(r["ms"] > 0 for r in out["chunk"]["rows"])
    assert [r["n"] for r in out["min_tokens"]["rows"]] == [1, 2, 4]
    assert [(r["pos0"], r["n"]) for r in out["prefill_map"]] == [(0, 256), (0, 1024),
                                                                 (4096, 256), (4096, 1024)]
    assert all(r["tflops"] > 0 for r in out["prefill_map"])
