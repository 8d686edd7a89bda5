"""Rotor compile (bivector -> rotor state) and sandwich application."""
from __future__ import annotations


def compile_bivector(bivector, n):
    raise NotImplementedError("rotor path not built yet")


def apply_rotor(state, x, n):
    raise NotImplementedError("rotor path not built yet")
