import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI of libzerollm_hip.so)")


@pytest.fixture(scope="session")
def tiny_files(tmp_path_factory):
    """The tiny qwen3 target / draft pair as GGUF files (Q8_0, d 512, 4 + 2 layers), written once per session."""
    from zerollm_amd import synth

    d = tmp_path_factory.mktemp("tiny")
    t, dr = synth.tiny_pair()
    tp, dp = str(d / "tiny_target.gguf"), str(d / "tiny_draft.gguf")
    synth.write_gguf(tp, t)
    synth.write_gguf(dp, dr)
    return tp, dp


@pytest.fixture(scope="session")
def close_files(tmp_path_factory):
    """The tiny pair with layer matrices of std 0.004 (embedding and head 0.02): the residual stream stays near the
    embedding, so the 2-layer draft agrees with the 4-layer target about 40 % of the time, greedy or sampled at
    temperature 0.7, and both the accept and the reject branches of a cycle run."""
    from zerollm_amd import synth

    d = tmp_path_factory.mktemp("close")
    t, dr = synth.tiny_pair(layer_std=0.004)
    tp, dp = str(d / "close_target.gguf"), str(d / "close_draft.gguf")
    synth.write_gguf(tp, t)
    synth.write_gguf(dp, dr)
    return tp, dp


@pytest.fixture(scope="session")
def gpu():
    """Initialise the GPU once (tests that use it are marked gpu)."""
    from zerollm_amd import model

    model.init(0)
    return model.device_info()
