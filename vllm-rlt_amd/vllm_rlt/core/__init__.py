"""Paged KV pool ownership (LAST_EXITED / SHARED planes)."""
