"""MoE layer surface (A side) and expert runner (F side)."""
