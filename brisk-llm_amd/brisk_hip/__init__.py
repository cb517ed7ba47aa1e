"""brisk_hip: the MI355X (gfx950) token loop of brisk-llm behind a C ABI.

``libbrisk_hip.so`` (built from ../csrc) is the product; this package is the
host-side mirror of the reference's Engine interface over it, plus the GGUF
reader/writer and the seeded synthetic models the benchmark runs.
"""
from .lib import BriskHipError, load  # noqa: F401
from .session import HipSession  # noqa: F401
