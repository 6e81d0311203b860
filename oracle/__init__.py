"""CPU oracle for the GLoRCQ hot path — test infrastructure only (see glorcq_oracle)."""
