"""Shared test setup: import paths, the `gpu` marker, seeded model files."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "rwkv-rsv_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle"), os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) to run")


# Small shapes for fast parity runs (head_size must be 64; k dims multiples of 128).
SMALL = dict(n_layer=2, c=256, vocab=1024, n_head=4, head_size=64, ffn=512, wm=64, am=64, vm=32, gm=128)


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("models")


def _model(model_dir, name, cfg, **kw):
    import synth
    path = os.path.join(str(model_dir), name + ".st")
    if not os.path.exists(path):
        synth.write_model(path, cfg, **kw)
    return path


@pytest.fixture(scope="session")
def small_f32(model_dir):
    return _model(model_dir, "small_f32", SMALL, seed=3)


@pytest.fixture(scope="session")
def small_f16(model_dir):
    return _model(model_dir, "small_f16", SMALL, seed=4, linear="f16", head="f16", emb="f16", lora="f16")


@pytest.fixture(scope="session")
def small_i8(model_dir):
    return _model(model_dir, "small_i8", SMALL, seed=5, linear="i8", head="i8")


@pytest.fixture(scope="session")
def small_i8_group(model_dir):
    return _model(model_dir, "small_i8g", SMALL, seed=6, linear="i8", head="i8", group_quant=True)


@pytest.fixture(scope="session")
def tiny_cfg1(model_dir):
    """Config 1: tiny RWKV-7, seed 0, fp32 N(0, 0.02^2)."""
    import synth
    return _model(model_dir, "tiny_cfg1", synth.TINY, seed=0)


def rel_rmse(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.sqrt(np.mean((a - b) ** 2)) / max(np.std(b), 1e-30))


def _cache_dir():
    return os.environ.get("RSV_BENCH_CACHE", "/tmp")


def three_b_model(kind):
    """The configs[3] 3B-shape model files (seed 1), cached like bench.py's:
    "i8" = int8 per-row-scale linears + int8 head (fp32 embedding in the file);
    "i8_f16" = int8 linears + fp16 embedding and fp16 head (the variant)."""
    import synth
    name, kw = {"i8": ("rsv_3b_i8_seed1.st", dict(linear="i8", head="i8")),
                "i8_f16": ("rsv_3b_i8_f16head_seed1.st", dict(linear="i8", head="f16", emb="f16"))}[kind]
    path = os.path.join(_cache_dir(), name)
    if not os.path.exists(path):
        tmp = path + ".tmp%d" % os.getpid()
        synth.write_model(tmp, synth.THREE_B, seed=1, **kw)
        os.replace(tmp, path)
    return path
