"""Operator facades over libkvip_hip.so."""
