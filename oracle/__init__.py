"""CPU checker for the verify path (test infrastructure; see oracle.h). Never imported by the product package."""
