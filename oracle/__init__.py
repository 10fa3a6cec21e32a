"""CPU oracle of the reference scan path (test infrastructure only)."""
