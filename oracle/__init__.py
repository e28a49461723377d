"""CPU oracle of the reference attention math (test infrastructure only)."""
