"""Test infrastructure only: the CPU restatement of the reference's int4 matmul arithmetic."""
