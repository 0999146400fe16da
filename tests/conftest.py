import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "llm-embed_amd"), os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libllmembed_hip.so")


@pytest.fixture(scope="session")
def gpu():
    """Initialise the HIP library; GPU tests fail loudly when it cannot."""
    import llmembed

    llmembed.init(0)
    return llmembed


@pytest.fixture(scope="session")
def small_spec():
    from llmembed import synth

    return synth.ModelSpec(n_layer=2)


@pytest.fixture(scope="session")
def full_spec():
    from llmembed import synth

    return synth.ModelSpec()
