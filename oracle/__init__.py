"""CPU oracle for the SwarmLoRA hot path (test infrastructure only; see
reference_path.py's header for who may import it)."""
