"""pytest configuration: the `gpu` marker, import paths and shared fixtures."""
import os
import shutil
import sys
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "qwen3-tts-hip_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on cuda:0)")


class _ModelCache:
    """Synthetic models written to disk once per session (the engine loads a model dir)."""

    def __init__(self):
        self.root = tempfile.mkdtemp(prefix="q3t_models_")
        self.models = {}

    def get(self, spec: str, seed: int = 0):
        from q3t import synth

        key = (spec, seed)
        if key not in self.models:
            model = synth.SyntheticModel.build(spec, seed)
            d = os.path.join(self.root, f"{spec}_{seed}")
            model.write(d)
            self.models[key] = (model, d)
        return self.models[key]

    def get_with_text(self, spec: str, seed: int = 0):
        """The same model written with its full text-embedding table, tokenizer files and the
        speech-tokenizer (codec) checkpoint: device text preparation, text inputs, audio."""
        from q3t import synth

        key = (spec, seed, "text")
        if key not in self.models:
            model, _ = self.get(spec, seed)
            d = os.path.join(self.root, f"{spec}_{seed}_text")
            model.write(d, text_embedding=True)
            synth.write_tokenizer(d)
            synth.write_codec(d, seed)
            self.models[key] = (model, d)
        return self.models[key]

    def drop(self, spec: str, seed: int = 0):
        item = self.models.pop((spec, seed), None)
        if item:
            shutil.rmtree(item[1], ignore_errors=True)

    def close(self):
        shutil.rmtree(self.root, ignore_errors=True)


@pytest.fixture(scope="session")
def models():
    cache = _ModelCache()
    yield cache
    cache.close()
