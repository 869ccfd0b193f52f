"""Model patches: attention forwards on the graph-ready paged cache."""
