"""Projection layout operators."""
