"""Scheduling passes over the tile IR (``warpir/passes/``)."""
