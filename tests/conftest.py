import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "glimpse-language_amd")
for p in (ROOT, os.path.join(ROOT, "tests"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def load_package():
    """The package directory name has a dash, so it is loaded by path under the name glimpse_language_amd."""
    if "glimpse_language_amd" in sys.modules:
        return sys.modules["glimpse_language_amd"]
    spec = importlib.util.spec_from_file_location("glimpse_language_amd", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["glimpse_language_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


@pytest.fixture(scope="session")
def gpu():
    """(torch, Context, Workspace) on cuda:0; the HIP library must be built (no fallback)."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    from glimpse_language_amd import bonsai_attn as ba
    ctx = ba.Context(0)
    ws = ba.Workspace(ctx, "cuda")
    yield torch, ctx, ws
    torch.cuda.synchronize()
    ctx.close()


def context_with(**env):
    """A bn_ctx on device 0 created with the given BONSAI_ATTN_* environment variables set (the context reads
    its knobs once, at creation); the environment is restored afterwards."""
    from glimpse_language_amd import bonsai_attn as ba
    old = {k: os.environ.get(k) for k in env}
    os.environ.update({k: str(v) for k, v in env.items()})
    try:
        return ba.Context(0)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v
