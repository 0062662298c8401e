"""ElasticBit CPU oracle (test infrastructure only; never imported by mlbricks_amd)."""
