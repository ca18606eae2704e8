"""CPU oracle of the batched token sampler (test infrastructure only)."""
