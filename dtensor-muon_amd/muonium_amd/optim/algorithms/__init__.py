"""Pluggable Muon algorithm variants, selected per param group via ``"algorithm"``."""

from .base import (
    BufferSpec,
    MuonAlgorithm,
    get_algorithm,
    orthogonalize_batch,
    orthogonalize_single,
    register_muon_algorithm,
    registered_algorithms,
    split_lr_scales,
)

# Importing these modules registers the built-in algorithms.
from .muon import MuonBaseline
from .normuon import NorMuon

__all__ = [
    "BufferSpec",
    "MuonAlgorithm",
    "MuonBaseline",
    "NorMuon",
    "get_algorithm",
    "orthogonalize_batch",
    "orthogonalize_single",
    "register_muon_algorithm",
    "registered_algorithms",
    "split_lr_scales",
]
