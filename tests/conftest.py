import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "squirrel-rs_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


# Small Llama-shaped models for parity tests: head_dim 64 as in Llama-3.2-1B,
# GQA group 4 (Llama) and 2, tied embeddings.
TINY = dict(n_layers=2, dim=512, ffn_dim=1024, n_heads=8, n_kv_heads=2, vocab=2048,
            context_length=4096)
TINY_G2 = dict(n_layers=2, dim=256, ffn_dim=512, n_heads=4, n_kv_heads=2, vocab=1000,
               context_length=2048)


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("models")


@pytest.fixture(scope="session")
def tiny_gguf(model_dir):
    """Path factory: tiny synthetic GGUF per (wtype, variant)."""
    import sqhip
    cache = {}

    def get(wtype="Q8_0", variant="g4", seed=7):
        key = (wtype, variant, seed)
        if key not in cache:
            dims = TINY if variant == "g4" else TINY_G2
            path = str(model_dir / f"tiny_{variant}_{wtype}_{seed}.gguf")
            sqhip.write_synthetic_gguf(path, wtype, seed=seed, **dims)
            cache[key] = path
        return cache[key]

    return get
