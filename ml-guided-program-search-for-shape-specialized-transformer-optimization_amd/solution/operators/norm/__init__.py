"""Residual operators."""
