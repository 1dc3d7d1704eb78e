"""yggdrasil_amd: Yggdrasil's int8 streaming inference step on AMD Instinct MI355X (gfx950).

The product is libygg_hip.so (HIP kernels + the C-ABI of include/ygg_hip.h) and the host class ``Yggdrasil``
(the reference's step/state API). ``fmt`` reads and writes the reference's YGG1 model files, ``synth`` makes the
seeded synthetic models and token streams of the benchmark configurations.
"""
from . import fmt, synth  # noqa: F401


def __getattr__(name):
    # the GPU class imports torch and opens the library lazily
    if name in ("Yggdrasil", "YggError", "load"):
        from . import inference
        return getattr(inference, name)
    raise AttributeError(name)
