"""slime_amd — MI355X (gfx950) multi-head neural-CA step of J0pari/Slime.

The compute lives in ``libslime_ca.so`` (hand-written HIP, C ABI in
``include/slime_ca.h``); this package is the host-side mirror used by the tests
and the benchmark. Importing it loads the library and fails loudly if it has
not been built: there is no CPU fallback. (The library is loaded on first use,
so ``python -m slime_amd.build`` can run before it exists.)
"""
from ._lib import SlimeError, load  # noqa: F401
from .ca import Pseudopod  # noqa: F401
from .pool import ComponentPool  # noqa: F401
from .synthetic import CONFIGS, CAConfig, make_params, make_state, round_bf16  # noqa: F401

