"""CPU restatement of the reference path. Test infrastructure only (see oracle.h)."""
