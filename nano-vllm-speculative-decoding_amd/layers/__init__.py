"""Drop-in layers of the verify hot path: paged attention and the speculative sampler."""
