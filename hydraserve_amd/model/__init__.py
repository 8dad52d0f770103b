"""Boundary types and the linear-layer dispatch of the reference's model runtime."""
