"""CPU oracle for the chunked delta-rule forward — test infrastructure only (see gdn_oracle)."""
