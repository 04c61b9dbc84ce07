"""Solution-owned runtimes (graph replay)."""

from .graph_replay import GraphReplay

__all__ = ["GraphReplay"]
