"""CPU oracle of the KV-cache migration path (test infrastructure only)."""
