"""CPU oracle for the MI355X kernel path (test infrastructure; see ref.py)."""
