"""TEST INFRASTRUCTURE ONLY: CPU oracle of the TurboAdam step (never imported by turboadam_amd)."""
