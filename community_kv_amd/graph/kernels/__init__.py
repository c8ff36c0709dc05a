"""Online graph-update workspace."""
