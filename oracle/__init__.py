"""CPU oracle of the LOCKS decode hot path (test infrastructure only)."""
