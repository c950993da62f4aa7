"""CPU oracle of the reference's prefix-reuse attention math (test infrastructure only)."""
