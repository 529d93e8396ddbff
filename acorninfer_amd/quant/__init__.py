"""Drop-in for acorninfer/quant: load-time RTN quantisation maths."""
