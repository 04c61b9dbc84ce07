"""Streamed long-sequence execution components, loaded only by streamed plans."""
