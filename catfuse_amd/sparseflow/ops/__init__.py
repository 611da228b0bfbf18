"""Pattern modules of the SparseFlow spatial backend (mirrors catfuse/sparseflow/ops/)."""
