"""CPU oracle for parity tests (test infrastructure only; never imported by chronicals_amd)."""
