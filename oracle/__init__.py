"""CPU oracle of the token loop (test infrastructure only)."""
