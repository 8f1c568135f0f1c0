"""CPU oracle of the reference learner spine (test infrastructure only)."""
