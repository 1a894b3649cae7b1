"""CPU oracle of the HiMuon step (test infrastructure only; see himuon_oracle)."""
