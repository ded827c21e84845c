"""CPU oracle for the GDN hot path (test infrastructure only)."""
