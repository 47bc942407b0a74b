"""Shared fixtures.

Tests marked ``gpu`` run the HIP path through the C ABI and compare it with ``oracle`` (the CPU
restatement of the reference).  Unmarked tests run on the CPU only: the oracle against the
reference's known answers and golden vectors, the file format, and the ABI's host-side behaviour.
"""
import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

# The box gives one GPU process a share of 16 cores; do not oversubscribe the CPU oracle.
os.environ.setdefault("OMP_NUM_THREADS", "16")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def lib():
    """The built libcudallm.so.  A missing build is an error, never a skip or a fallback."""
    from cudallm_amd import engine as E
    return E.lib()


@pytest.fixture(scope="session")
def gpu(lib):
    """Fails loudly when a gpu test runs without a visible GPU."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test without a visible GPU")
    name = torch.cuda.get_device_properties(0).gcnArchName
    print(f"[gpu] device 0: {torch.cuda.get_device_name(0)} ({name})", flush=True)
    return name


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    d = os.environ.get("CUDALLM_TEST_MODELS")
    if d:
        Path(d).mkdir(parents=True, exist_ok=True)
        return Path(d)
    return tmp_path_factory.mktemp("models")


# The engine tests' model files: seeded Llama-3.2-1B-shaped weights with random norm weights (so a
# wrong norm index shows) and a header that allows 16384 positions (contexts past 8192).
TEST_MODEL_SEED = 1234
TEST_MODEL_MAX_SEQ = 16384


@pytest.fixture(scope="session")
def model_path(gpu, model_dir):
    """model_path(wd) -> path of the shared test model for weight type wd, written on first use."""
    from cudallm_amd import synth
    cache = {}

    def get(wd):
        if wd not in cache:
            p = model_dir / f"synth_seed{TEST_MODEL_SEED}_{wd}_norm_ms{TEST_MODEL_MAX_SEQ}.cudallm"
            if not p.exists():
                print(f"[model] writing {p}", flush=True)
                synth.write_model(p, wd, seed=TEST_MODEL_SEED, max_seq_len=TEST_MODEL_MAX_SEQ, norm="random")
            cache[wd] = p
        return cache[wd]
    return get
