"""CPU oracle of nimbus-infer-rs src/sampler.rs (test infrastructure only)."""
