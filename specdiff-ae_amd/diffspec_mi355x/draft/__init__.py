"""Acceptance of a verified draft tree."""
