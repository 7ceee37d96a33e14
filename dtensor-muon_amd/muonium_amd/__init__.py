"""muonium_amd: MI355X-native Muon optimizer step (drop-in for muonium's API).

The Python layer keeps muonium's optimizer / algorithm-plugin surface; every
Muon-family step runs hand-written gfx950 kernels from libmuon_amd.so through a C ABI
(include/muon_amd.h).
"""

from .optim import (
    BufferSpec,
    Muon,
    Muon4bit,
    Muon8bit,
    MuonAlgorithm,
    MuonFp8,
    MuonLP,
    get_algorithm,
    register_muon_algorithm,
    registered_algorithms,
)
from .orthogonalize import OrthogonalizationStrategy

__all__ = [
    "BufferSpec",
    "Muon",
    "Muon4bit",
    "Muon8bit",
    "MuonAlgorithm",
    "MuonFp8",
    "MuonLP",
    "OrthogonalizationStrategy",
    "get_algorithm",
    "register_muon_algorithm",
    "registered_algorithms",
]
