"""Host-side kernel modules of the paged MHA operator."""
