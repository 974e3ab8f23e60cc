"""Request state and KV-page bookkeeping of the verification round."""
