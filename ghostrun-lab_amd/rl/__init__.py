"""Host side of the MI355X batched NES environment step (drop-in for the reference's rl/ package surface)."""
