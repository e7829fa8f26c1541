"""CPU oracle of the paged-attention path (test infrastructure only)."""
