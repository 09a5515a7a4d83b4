/* placeholder: filled in with the attention oracle */
