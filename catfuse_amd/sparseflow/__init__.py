"""SparseFlow side of CATFuse-SF on gfx950: prescan, routing constants and
the multi-step LIF launcher (mirrors catfuse/sparseflow/)."""
