"""CPU oracle of the KV hot path — test infrastructure only (see kv_oracle.py)."""
