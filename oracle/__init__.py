"""FP64 CPU oracle -- test infrastructure only (see oracle/sejong_oracle.c)."""
