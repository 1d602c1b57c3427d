"""CPU oracle for the MoC hot path: test infrastructure, never the product path."""
