"""Online handoff primitives: block packing, fused install, leases, pipeline."""
