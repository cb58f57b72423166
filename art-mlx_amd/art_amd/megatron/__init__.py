"""Mirrors of art.megatron modules on the MI355X path."""
