"""Byte budget (Arena) and weight sources feeding the streaming path."""
