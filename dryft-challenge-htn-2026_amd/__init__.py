"""MI355X-native (gfx950) decode step of a Qwen3-shape greedy-decode engine.

Host side: :class:`engine.Engine` (reference API: ``Engine(model_path)``, ``generate``),
:class:`hipops.HipOps` (the reference's ops interface over the HIP kernels), ``synth`` (seeded
random-init checkpoints). Device side: ``csrc/*.hip`` -> ``libdryft_decode.so`` (C ABI in
``include/dryft_decode.h``).

The directory name is not a Python identifier; tests and tools import it under the alias
``dryft_amd`` (see ``load_package`` in ``__graft_entry__.py``).
"""
from . import synth  # noqa: F401
from ._lib import LIB_PATH, exported_symbols, lib  # noqa: F401
