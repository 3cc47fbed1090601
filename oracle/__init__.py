"""CPU oracle of the decode-attention path (test infrastructure only)."""
