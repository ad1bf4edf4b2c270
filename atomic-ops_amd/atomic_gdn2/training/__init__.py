"""Training-side helpers around the operator (reference ``atomic_gdn2/training``)."""
