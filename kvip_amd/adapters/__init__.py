"""Serving-engine adapters of the LIFetch path."""
