"""GPU test of the build's own driver, ``mega-kernel_amd/model.py``: the reference validates its
kernel only by running its driver end to end (/root/reference/model.py:95-136), so the driver's four
paths run here on the 0.6B shape for a few tokens -- the host greedy loop and the device-side loop
(``--device-loop``), each after the Transformers prefill plus cache copy and after the native
prefill (``--native-prefill``). Each must end with a clean device status, and its tokens must equal
``decode_steps(generate=True)`` replayed from the cache the prefill left."""
import pytest
import torch

pytestmark = pytest.mark.gpu

NEW = 6
ARGS = ["--shape", "qwen3-0.6b", "--prompt", "32", "--max-seq", "128", "--new", str(NEW)]


@pytest.fixture(scope="module")
def driver():
    import model
    return model


@pytest.mark.parametrize("flags", [[], ["--device-loop"], ["--native-prefill"], ["--device-loop", "--native-prefill"]],
                         ids=["host-loop", "device-loop", "native-prefill", "native-prefill-device-loop"])
def test_driver_matches_decode_steps(driver, flags):
    import megakernel
    r = driver.run(ARGS + flags, keep_prefill_cache=True)
    assert r["status"] == 0
    assert len(r["generated"]) == NEW and all(0 <= t < 151936 for t in r["generated"])
    kernel = megakernel.load()
    inp = r["inputs"]
    kd, vd = (t.clone() for t in r["prefill_cache"])
    tokens = torch.zeros(NEW, dtype=torch.int32, device="cuda:0")
    tokens[0] = r["first_token"]
    kernel.decode_steps(tokens, NEW - 1, True, inp["embed"], inp["embed"], inp["final_norm"], inp["layer_weights"],
                        inp["cos"], inp["sin"], kd, vd, r["prompt"], inp["max_seq"])
    assert tokens.tolist() == r["generated"], (tokens.tolist(), r["generated"])
    assert kernel.status() == 0


def test_driver_paths_agree(driver):
    """The host loop and the device loop generate the same tokens after the same prefill, and the
    command line reports success (exit status 0)."""
    a = driver.run(ARGS)
    b = driver.run(ARGS + ["--device-loop"])
    assert a["generated"] == b["generated"]
    assert driver.main(ARGS + ["--native-prefill", "--device-loop"]) == 0
