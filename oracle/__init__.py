"""CPU oracle for the Jules kernel path -- test infrastructure only (see jules_oracle.h)."""
