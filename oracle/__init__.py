"""CPU oracle of the token loop — test infrastructure only (see oracle.h)."""
