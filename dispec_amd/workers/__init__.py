"""Callers of the KV path kept from the reference: escalation (cross-model transfer)."""
